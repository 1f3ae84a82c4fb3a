"""GPU parity of the prefill path: the MFMA Matmul (m > 1, transposeB, f16 and
bf16 with f32 accumulation; Matmul.swift:175-196, MPPMatmul.metal:19-91)
against the oracle's Matmul loop (KernelsTests.swift:239-267 order)."""
import numpy as np
import pytest

import oracle as O
from conftest import assert_out
from gpu_util import EPS, download, gpu_env, rounded, upload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def _gemm(env, a, b, at, ot):
    pa, lib, stream, enc = env
    M, K = a.shape
    N = b.shape[0]
    c = pa.Tensor.empty([M, N], ot)
    k = pa.Kernels.Matmul(upload(pa, a, at), upload(pa, b, at), c, True)
    enc.encode(k)
    stream.synchronize()
    return download(c, stream).reshape(M, N), k


@pytest.mark.parametrize("at,ot", [("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32")])
@pytest.mark.parametrize("M,K,N", [(128, 64, 128), (130, 200, 90), (256, 1024, 384), (1, 64, 300), (300, 8, 129)])
def test_mfma_matmul_vs_oracle(env, at, ot, M, K, N):
    a = rounded(O.normal(M + K, (M, K)), at)
    b = rounded(O.normal(N + K, (N, K), std=0.02), at)
    got, k = _gemm(env, a, b, at, ot)
    if M > 1:
        assert k.function_names[0].startswith(f"matmul_mfma_{at}_{at}_{ot}_t")
    ref = O.matmul(a, b, M, K, N, True).reshape(M, N)
    # inputs exact in their dtype, f32 accumulation in another order: 1e-5
    # for f32 outputs, else the 16-bit bar plus the store's rounding
    assert_out(got, ref, 1e-5 if ot == "f32" else EPS[at], ot, f"mfma gemm {at}->{ot} {M}x{K}x{N}")


@pytest.mark.parametrize("at", ["f16", "bf16"])
def test_mfma_matmul_integer_exact(env, at):
    # small integers: every product and partial sum is exact in f32, so the
    # result is exact whatever the summation order: pins every fragment index
    rng = np.random.default_rng(7)
    M, K, N = 192, 320, 160
    a = rng.integers(-4, 5, (M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (N, K)).astype(np.float32)
    got, _ = _gemm(env, a, b, at, "f32")
    np.testing.assert_array_equal(got, (a.astype(np.int64) @ b.T.astype(np.int64)).astype(np.float32))


@pytest.mark.parametrize("M,K,N", [(2048, 3072, 9216), (2048, 3072, 24576), (2048, 24576, 3072)])
def test_mfma_matmul_config5_shapes_sampled(env, M, K, N):
    # BASELINE config 5 (Gemma-7B prefill, f16): QKV, gate/up, down. The
    # oracle checks 6 rows, including the first and the last tile rows.
    pa, lib, stream, enc = env
    ta, tb = pa.Tensor.empty([M, K], "f16"), pa.Tensor.empty([N, K], "f16")
    lib.fill_normal(ta, 11, stream=stream)
    lib.fill_normal(tb, 12, std=0.02, stream=stream)
    c = pa.Tensor.empty([M, N], "f16")
    k = pa.Kernels.Matmul(ta, tb, c, True)
    enc.encode(k)
    stream.synchronize()
    assert k.function_names[0].startswith("matmul_mfma_f16_f16_f16_t")
    rows = [0, 1, 127, 128, M // 2 + 3, M - 1]
    a = download(ta, stream).reshape(M, K)[rows]
    b = download(tb, stream).reshape(N, K)
    got = download(c, stream).reshape(M, N)[rows]
    ref = O.matmul(a, b, len(rows), K, N, True).reshape(len(rows), N)
    assert_out(got, ref, EPS["f16"], "f16", f"config5 {M}x{K}x{N}")
