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


def _name(at, ot, M, N):
    # A staged in LDS at >= 512 tiles of 16 rows of B; else 16-row blocks
    # (_r16) when 32-row blocks would be fewer than the CUs (MI355X: 256)
    suffix = "_lds" if -(-N // 16) >= 512 else ("_r16" if -(-N // 32) < 256 else "")
    return f"matmul_skinny_{at}_{at}_{ot}_m{16 * (-(-M // 16))}" + suffix


@pytest.mark.parametrize("at,ot", [("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32")])
@pytest.mark.parametrize("M,K,N", [(2, 64, 67), (8, 2304, 9216), (8, 2304, 2304), (16, 136, 300), (17, 520, 129),
                                   (33, 256, 1000), (48, 2048, 64), (64, 3072, 512), (5, 8, 33), (63, 40, 31),
                                   (8, 9216, 2304), (32, 2304, 4096), (40, 1032, 8200), (2, 8, 8200),
                                   (48, 1000, 8195), (64, 520, 9000), (16, 4104, 8192), (8, 2304, 8176)])
def test_skinny_matmul_vs_oracle(env, at, ot, M, K, N):
    a = rounded(O.normal(M * 7 + K, (M, K)), at)
    b = rounded(O.normal(N * 3 + K, (N, K), std=0.02), at)
    got, k = _gemm(env, a, b, at, ot, guard=64)
    assert k.function_names == [_name(at, ot, M, N)]
    ref = O.matmul(a, b, M, K, N, True).reshape(M, N)
    if ot == "f32":
        # inputs exact in their dtype, f32 sums in another order: 1e-5 of the
        # sum of the terms' magnitudes (an element that cancels to near zero
        # keeps the rounding of its large partial sums)
        mag = np.abs(a).astype(np.float64) @ np.abs(b).T.astype(np.float64)
        err = np.abs(got.astype(np.float64) - ref)
        assert (err <= 1e-5 * mag).all(), f"skinny gemm {at}->f32 {M}x{K}x{N}: max err/mag {np.max(err / mag):.3e}"
    else:
        # the 16-bit bar plus the store's rounding
        assert_out(got, ref, EPS[at], ot, f"skinny gemm {at}->{ot} {M}x{K}x{N}")


@pytest.mark.parametrize("at", ["f16", "bf16"])
@pytest.mark.parametrize("M,K,N", [(3, 320, 160), (16, 1000, 64), (40, 96, 250), (64, 4104, 96), (16, 520, 9000),
                                   (61, 264, 8230), (33, 1000, 8195), (2, 264, 16384), (64, 2056, 8192), (8, 8, 8200)])
def test_skinny_matmul_integer_exact(env, at, M, K, N):
    # small integers: every product and partial sum is exact in f32, so the
    # result is exact whatever the order (K-split over waves, LDS sum): pins
    # every fragment index, the row clamps and the K tail
    rng = np.random.default_rng(M * 1000 + K)
    a = rng.integers(-4, 5, (M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (N, K)).astype(np.float32)
    got, k = _gemm(env, a, b, at, "f32", guard=16)
    assert k.function_names == [_name(at, "f32", M, N)]
    np.testing.assert_array_equal(got, (a.astype(np.int64) @ b.T.astype(np.int64)).astype(np.float32))
