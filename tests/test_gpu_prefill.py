"""GPU parity of the prefill path: the MFMA Matmul (m > 1, transposeB, f16 and
bf16 with f32 accumulation; Matmul.swift:175-196, MPPMatmul.metal:19-91)
against the oracle's Matmul loop (KernelsTests.swift:239-267 order)."""
import numpy as np
import pytest

import oracle as O
from conftest import assert_out
from gpu_util import EPS, TAG, download, gpu_env, rounded, upload

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
        assert k.function_names[0].startswith(f"matmul_mfma_{at}_{at}_{ot}_")
    ref = O.matmul(a, b, M, K, N, True).reshape(M, N)
    # inputs exact in their dtype, f32 accumulation in another order: 1e-5
    # for f32 outputs, else the 16-bit bar plus the store's rounding
    assert_out(got, ref, 1e-5 if ot == "f32" else EPS[at], ot, f"mfma gemm {at}->{ot} {M}x{K}x{N}")


@pytest.mark.parametrize("at,ot", [("f16", "f16"), ("bf16", "bf16"), ("bf16", "f32")])
@pytest.mark.parametrize("M,K,N", [(128, 64, 128), (130, 200, 90), (256, 1024, 384), (8, 2304, 1000), (300, 8, 129),
                                   (64, 72, 4097)])
def test_mfma_matmul_b_not_transposed_vs_oracle(env, at, ot, M, K, N):
    # a [K, N] B (the reference's mpp_matmul without _tb, Matmul.swift:203-214):
    # B^T into scratch by transpose2d_b16 (ragged 64 x 64 tiles included),
    # then the transposed-B matrix-core route (MFMA tiles, or skinny at M <= 64)
    pa, lib, stream, enc = env
    a = rounded(O.normal(M + K + 1, (M, K)), at)
    b = rounded(O.normal(N + K + 2, (K, N), std=0.02), at)
    c = pa.Tensor.empty([M, N], ot)
    k = pa.Kernels.Matmul(upload(pa, a, at), upload(pa, b, at), c, False)
    assert k.function_names[0] == "transpose2d_b16"
    assert k.function_names[1].startswith(("matmul_mfma_", "matmul_skinny_"))
    enc.encode(k)
    stream.synchronize()
    got = download(c, stream).reshape(M, N)
    ref = O.matmul(a, b, M, K, N, False).reshape(M, N)
    assert_out(got, ref, 1e-5 if ot == "f32" else EPS[at], ot, f"gemm B [K, N] {at}->{ot} {M}x{K}x{N}")


@pytest.mark.parametrize("at,bt", [("f32", "f32"), ("f32", "bf16"), ("bf16", "f32")])
@pytest.mark.parametrize("tb", [True, False])
@pytest.mark.parametrize("M,K,N", [(2, 4, 4), (130, 200, 92), (256, 1028, 384), (300, 36, 132), (1024, 3072, 1024)])
def test_mfma_f32_matmul_vs_oracle(env, at, bt, tb, M, K, N):
    # f32 output with an f32 operand (the reference's MPP f32 combinations,
    # Matmul.swift:203-214) on v_mfma_f32_16x16x4_f32: bf16 operands widen
    # exactly, products and sums in f32 in another order than the oracle's,
    # so the f32 bar; ragged tiles, K not a multiple of the 16-value step
    pa, lib, stream, enc = env
    a = rounded(O.normal(M + K + 3, (M, K)), at)
    b = rounded(O.normal(N + K + 4, (N, K) if tb else (K, N), std=0.05), bt)
    c = pa.Tensor.empty([M, N], "f32")
    k = pa.Kernels.Matmul(upload(pa, a, at), upload(pa, b, bt), c, tb)
    assert k.function_names == [f"matmul_mfma_{at}_{bt}_f32" + ("_tb" if tb else "")]
    enc.encode(k)
    stream.synchronize()
    got = download(c, stream).reshape(M, N)
    ref = O.matmul(a, b, M, K, N, tb).reshape(M, N)
    assert_out(got, ref, 1e-5, "f32", f"f32 mfma gemm {at}x{bt} tb={tb} {M}x{K}x{N}")


def test_mfma_f32_matmul_integer_exact(env):
    # small integers: every product and partial sum is exact in f32, so the
    # result is exact whatever the order; pins the k order of the 16-value
    # step and the transposed B staging
    pa, lib, stream, enc = env
    rng = np.random.default_rng(31)
    M, K, N = 200, 516, 260
    a = rng.integers(-8, 9, (M, K)).astype(np.float32)
    b = rng.integers(-8, 9, (K, N)).astype(np.float32)
    c = pa.Tensor.empty([M, N], "f32")
    k = pa.Kernels.Matmul(upload(pa, a, "f32"), upload(pa, b, "f32"), c, False)
    assert k.function_names == ["matmul_mfma_f32_f32_f32"]
    enc.encode(k)
    stream.synchronize()
    np.testing.assert_array_equal(download(c, stream).reshape(M, N), (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))


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


TILES = [f"{f}{t}" for f in "ed" for t in ("256x384", "256x256", "128x128", "128x256", "128x192")] + ["e256x288"]


@pytest.mark.parametrize("tile", TILES)
def test_mfma_matmul_every_tile_integer_exact(env, monkeypatch, tile):
    # every direct-copy tile (POPCORN_GEMM_TILE) on ragged M and N, with 1, 2
    # and 5 K stages (64 deep for the whole-line "e" tiles, 32 for "d"):
    # small integers make the f32 result exact in any order, so every copy
    # offset, LDS slot and fragment index is pinned; rows and columns past
    # M and N read zeros or clamped rows and are not stored
    monkeypatch.setenv("POPCORN_GEMM_TILE", tile)
    rng = np.random.default_rng(21)
    stage = 64 if tile[0] == "e" else 32
    for at in ("f16", "bf16"):
        for M, N, stages in [(300, 400, 1), (517, 131, 2), (264, 392, 5)]:
            K = stage * stages
            a = rng.integers(-4, 5, (M, K)).astype(np.float32)
            b = rng.integers(-4, 5, (N, K)).astype(np.float32)
            got, k = _gemm(env, a, b, at, "f32")
            assert k.function_names == [f"matmul_mfma_{at}_{at}_f32_{tile}"]
            np.testing.assert_array_equal(got, (a.astype(np.int64) @ b.T.astype(np.int64)).astype(np.float32),
                                          err_msg=f"{tile} {at} {M}x{K}x{N}")


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("at,ot", [("f16", "f16"), ("bf16", "bf16")])
def test_mfma_matmul_every_tile_vs_oracle(env, monkeypatch, tile, at, ot):
    monkeypatch.setenv("POPCORN_GEMM_TILE", tile)
    M, N = 390, 270
    K = 448 if tile[0] == "e" else 416
    a = rounded(O.normal(M + K + 1, (M, K)), at)
    b = rounded(O.normal(N + K + 1, (N, K), std=0.02), at)
    got, k = _gemm(env, a, b, at, ot)
    assert k.function_names == [f"matmul_mfma_{at}_{at}_{ot}_{tile}"]
    ref = O.matmul(a, b, M, K, N, True).reshape(M, N)
    assert_out(got, ref, EPS[at], ot, f"mfma gemm {tile} {at}->{ot} {M}x{K}x{N}")


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
    assert k.function_names[0].startswith(("matmul_mfma_f16_f16_f16_", "matmul_mfma_f16_splitk_"))
    rows = [0, 1, 127, 128, M // 2 + 3, M - 1]
    a = download(ta, stream).reshape(M, K)[rows]
    b = download(tb, stream).reshape(N, K)
    got = download(c, stream).reshape(M, N)[rows]
    ref = O.matmul(a, b, len(rows), K, N, True).reshape(len(rows), N)
    assert_out(got, ref, EPS["f16"], "f16", f"config5 {M}x{K}x{N}")


@pytest.mark.parametrize("at", ["f16", "bf16"])
@pytest.mark.parametrize("K,form", [(16384, "e"), (16640, "d")])
def test_mfma_matmul_split_k_integer_exact(env, at, K, form):
    # 32 ragged 256 x 384 tiles x 8 K splits (of 2048: whole-line stages of
    # 64; of 2080: 64-byte-row stages of 32): small integers keep every
    # partial sum exact, so the f32 result is exact whatever the split
    pa, lib, stream, enc = env
    rng = np.random.default_rng(13)
    M, N = 2000, 1500
    a = rng.integers(-4, 5, (M, K)).astype(np.float32)
    b = rng.integers(-4, 5, (N, K)).astype(np.float32)
    got, k = _gemm(env, a, b, at, "f32")
    assert k.function_names == [f"matmul_mfma_{at}_splitk_{form}256x384", "matmul_splitk_reduce_f32"]
    # |sums| <= 16 K < 2^24: exact in f64 (BLAS) and in f32
    np.testing.assert_array_equal(got, (a.astype(np.float64) @ b.T.astype(np.float64)).astype(np.float32))


@pytest.mark.parametrize("at,ot", [("f16", "f16"), ("bf16", "bf16"), ("bf16", "f32")])
def test_mfma_matmul_split_k_vs_oracle(env, at, ot):
    # the split-K reduction rounds once to the output dtype; oracle on sampled rows
    pa, lib, stream, enc = env
    M, K, N = 2000, 16384, 1500
    a = rounded(O.normal(5, (M, K)), at)
    b = rounded(O.normal(6, (N, K), std=0.02), at)
    got, k = _gemm(env, a, b, at, ot)
    assert k.function_names[1] == f"matmul_splitk_reduce_{ot}"
    rows = [0, 255, 256, 1000, 1791, 1792, M - 1]
    ref = O.matmul(a[rows], b, len(rows), K, N, True).reshape(len(rows), N)
    if ot == "f32":
        # f32 sums of 16384 terms in another order: the bar is 1e-5 of the
        # sum of the terms' magnitudes (an element that cancels to near zero
        # keeps the rounding of its large partial sums)
        mag = np.abs(a[rows]).astype(np.float64) @ np.abs(b).T.astype(np.float64)
        err = np.abs(got[rows].astype(np.float64) - ref)
        assert (err <= 1e-5 * mag).all(), f"split-K gemm {at}->f32: max err/mag {np.max(err / mag):.3e}"
    else:
        assert_out(got[rows], ref, EPS[at], ot, f"split-K gemm {at}->{ot}")


# ---- tiled (MFMA) FlashAttention prefill ---------------------------------------

def _attend(env, q, k, v, dtype, out_dtype, scale, mask):
    pa, lib, stream, enc = env
    B, Nq, Sq, Hd = q.shape
    Nkv, cap = k.shape[1], k.shape[2]
    to = pa.Tensor.empty([B, Nq, Sq, Hd], out_dtype)
    kern = pa.Kernels.FlashAttention(upload(pa, q, dtype), upload(pa, k, dtype), upload(pa, v, dtype), out=to,
                                     scale=scale, mask=mask, batch=B, query_heads=Nq, kv_heads=Nkv, query_len=Sq,
                                     key_len=cap, head_dim=Hd)
    enc.encode(kern)
    stream.synchronize()
    return download(to, stream), kern


MASKS = {"causal": (0, -1), "bidirectional": (2, -1), "window40": (1, 40)}


@pytest.fixture(params=["rows16", "rows32"])
def rows(request, monkeypatch):
    # Hd 128 and 256 run the 16-rows-per-wave kernel unless
    # POPCORN_FA_ROWS=32 selects the 32-row one: both are checked
    if request.param == "rows32":
        monkeypatch.setenv("POPCORN_FA_ROWS", "32")
    else:
        monkeypatch.delenv("POPCORN_FA_ROWS", raising=False)
    return request.param


def _tiled(dtype, ot, Hd, rows):
    kind = "tiled16" if Hd in (128, 256) and rows == "rows16" else "tiled"
    return f"flash_attention_{kind}_{dtype}_{ot}_d{Hd}"


def _paired(dtype, ot, Hd, rows):
    # paired causal tiles (at most one tile per CU): the second block of a
    # pair merges the split tile itself, no merge kernel
    return [_tiled(dtype, ot, Hd, rows)]


@pytest.mark.parametrize("dtype,ot", [("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32")])
@pytest.mark.parametrize("B,Nq,Nkv,Sq,Sk,Hd,mask", [
    (1, 2, 1, 64, 64, 64, "causal"),
    (2, 4, 2, 130, 200, 128, "causal"),        # Sq < Sk: posQ = Sk - Sq + i; ragged tiles
    (1, 2, 2, 96, 96, 256, "bidirectional"),
    (1, 2, 1, 128, 160, 64, "window40"),
    (1, 1, 1, 32, 32, 256, "causal"),
    (2, 4, 2, 130, 200, 256, "causal"),        # GQA, Sq < Sk, ragged tiles at Hd 256
    (1, 2, 1, 128, 160, 256, "window40"),
])
def test_tiled_attention_vs_oracle(env, rows, dtype, ot, B, Nq, Nkv, Sq, Sk, Hd, mask):
    pa = env[0]
    kind, window = MASKS[mask]
    q = rounded(O.normal(Sq + Hd, (B, Nq, Sq, Hd)), dtype)
    k = rounded(O.normal(Sk + Hd + 1, (B, Nkv, Sk, Hd)), dtype)
    v = rounded(O.normal(Sk + Hd + 2, (B, Nkv, Sk, Hd)), dtype)
    pm = pa.AttentionMask(kind, window)
    scale = 1 / np.sqrt(Hd)
    got, kern = _attend(env, q, k, v, dtype, ot, scale, pm)
    assert kern.function_names == [_tiled(dtype, ot, Hd, rows)]
    ref = O.attention_naive(q, k, v, scale, mask_kind=kind, window=window)
    assert not np.isnan(got).any()
    # softmax weights enter the P.V product in the input dtype (the matrix
    # cores multiply 16-bit operands: f16 rounds them to 11 bits, bf16 carries
    # a high part and a remainder); the normaliser sums the same weights
    assert_out(got, ref, EPS[dtype], ot, f"tiled attention {dtype}->{ot} {mask} Sq={Sq} Sk={Sk} Hd={Hd}")


def _tiled_any(dtype, ot, Hd, rows):
    # the kernel of a head dim padded to 64, 128, 256 or 512
    hdp = 64 if Hd <= 64 else 128 if Hd <= 128 else 256 if Hd <= 256 else 512
    kind = "tiled16" if hdp == 512 or (hdp in (128, 256) and rows == "rows16") else "tiled"
    return f"flash_attention_{kind}_{dtype}_{ot}_d{hdp}"


@pytest.mark.parametrize("dtype,ot", [("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32")])
@pytest.mark.parametrize("B,Nq,Nkv,Sq,Sk,Hd,mask", [
    (1, 2, 1, 130, 200, 512, "causal"),        # Gemma-4 global head dim: GQA, Sq < Sk, ragged tiles
    (1, 2, 2, 96, 96, 512, "bidirectional"),
    (1, 2, 1, 128, 160, 512, "window40"),
    (1, 4, 2, 300, 300, 320, "causal"),        # padded to 512
    (2, 4, 2, 70, 90, 80, "causal"),           # padded to 128
    (1, 2, 1, 64, 100, 192, "window40"),       # padded to 256
    (1, 2, 2, 40, 40, 40, "bidirectional"),    # padded to 64
    (1, 2, 1, 33, 33, 8, "causal"),
])
def test_tiled_attention_any_head_dim_vs_oracle(env, rows, dtype, ot, B, Nq, Nkv, Sq, Sk, Hd, mask):
    # the matrix-core route for every 16-bit head dim up to 512 in 16-byte
    # rows (the reference's MPP route takes any Hd <= 512 with Sq >= 32,
    # FlashAttention.swift:109-113, in hd256/hd512 buckets :305-311): the
    # kernel's dims past Hd are zeros and its stores stop at Hd. The output
    # starts as NaN with guard rows after it, so a skipped or stray store fails.
    pa, lib, stream, enc = env
    kind, window = MASKS[mask]
    q = rounded(O.normal(Sq + Hd + 5, (B, Nq, Sq, Hd)), dtype)
    k = rounded(O.normal(Sk + Hd + 6, (B, Nkv, Sk, Hd)), dtype)
    v = rounded(O.normal(Sk + Hd + 7, (B, Nkv, Sk, Hd)), dtype)
    scale = 1 / np.sqrt(Hd)
    n = B * Nq * Sq * Hd
    buf = upload(pa, np.full(n + 64, np.nan, np.float32), ot)
    to = buf.view([B, Nq, Sq, Hd])
    kern = pa.Kernels.FlashAttention(upload(pa, q, dtype), upload(pa, k, dtype), upload(pa, v, dtype), out=to,
                                     scale=scale, mask=pa.AttentionMask(kind, window), batch=B, query_heads=Nq,
                                     kv_heads=Nkv, query_len=Sq, key_len=Sk, head_dim=Hd)
    assert kern.function_names == [_tiled_any(dtype, ot, Hd, rows)]
    enc.encode(kern)
    stream.synchronize()
    out = download(buf, stream)
    assert np.isnan(out[n:]).all(), "stores past the output"
    got = out[:n].reshape(B, Nq, Sq, Hd)
    assert not np.isnan(got).any()
    ref = O.attention_naive(q, k, v, scale, mask_kind=kind, window=window)
    assert_out(got, ref, EPS[dtype], ot, f"tiled attention {dtype}->{ot} {mask} Sq={Sq} Sk={Sk} Hd={Hd}")


@pytest.mark.parametrize("B,Nq,Nkv,Sq,Sk,cap,Hd,mask", [
    (1, 2, 1, 64, 64, 64, 64, "causal"),
    (2, 4, 2, 130, 200, 207, 128, "causal"),     # GQA, Sq < Sk, ragged tiles, key capacity > Sk
    (1, 2, 2, 96, 96, 96, 256, "bidirectional"),
    (1, 2, 1, 128, 160, 160, 64, "window40"),
    (1, 2, 1, 130, 200, 200, 512, "causal"),
    (1, 2, 2, 96, 96, 96, 512, "bidirectional"),
    (1, 2, 1, 128, 160, 160, 512, "window40"),
    (1, 4, 2, 300, 300, 300, 320, "causal"),     # padded to 512
    (2, 4, 2, 70, 90, 90, 80, "causal"),         # padded to 128
    (1, 2, 1, 64, 100, 100, 192, "window40"),    # padded to 256
    (1, 2, 2, 40, 40, 40, 36, "bidirectional"),  # padded to 64
    (1, 2, 1, 33, 33, 33, 4, "causal"),
])
def test_tiled_attention_f32_vs_oracle(env, B, Nq, Nkv, Sq, Sk, cap, Hd, mask):
    # f32 Q, K, V on v_mfma_f32_16x16x4_f32, the role of the reference's
    # mpp_flash_attention_f32 (FlashAttention.swift:368-376) for any Hd <= 512
    # in 16-byte rows: f32 products and sums in another order than the
    # oracle's, so the f32 bar. The output starts as NaN with guard elements
    # after it, so a skipped or stray store fails.
    pa, lib, stream, enc = env
    kind, window = MASKS[mask]
    q = O.normal(Sq + Hd + 15, (B, Nq, Sq, Hd))
    k = O.normal(Sk + Hd + 16, (B, Nkv, cap, Hd))
    v = O.normal(Sk + Hd + 17, (B, Nkv, cap, Hd))
    scale = 1 / np.sqrt(Hd)
    n = B * Nq * Sq * Hd
    buf = upload(pa, np.full(n + 64, np.nan, np.float32), "f32")
    kern = pa.Kernels.FlashAttention(upload(pa, q, "f32"), upload(pa, k, "f32"), upload(pa, v, "f32"),
                                     out=buf.view([B, Nq, Sq, Hd]), scale=scale, mask=pa.AttentionMask(kind, window),
                                     batch=B, query_heads=Nq, kv_heads=Nkv, query_len=Sq, key_len=Sk, head_dim=Hd,
                                     key_capacity=cap)
    hdp = 64 if Hd <= 64 else 128 if Hd <= 128 else 256 if Hd <= 256 else 512
    assert kern.function_names == [f"flash_attention_tiled16_f32_f32_d{hdp}"]
    enc.encode(kern)
    stream.synchronize()
    out = download(buf, stream)
    assert np.isnan(out[n:]).all(), "stores past the output"
    got = out[:n].reshape(B, Nq, Sq, Hd)
    assert not np.isnan(got).any()
    ref = O.attention_naive(q, k, v, scale, mask_kind=kind, window=window, key_len=Sk)
    assert_out(got, ref, EPS["f32"], "f32", f"tiled attention f32 {mask} Sq={Sq} Sk={Sk} Hd={Hd}")


@pytest.mark.parametrize("Hd,Nq,Nkv", [(128, 8, 8), (512, 4, 2)])
def test_tiled_attention_f32_sampled(env, Hd, Nq, Nkv):
    # f32 prefill at 2048 tokens, causal, with scores of standard deviation
    # 4.5 natural-log units (inputs x 1.5, scale 1/sqrt(Hd) x 2), so the
    # running max moves past the lazy-rescale gap; sampled query rows against
    # the oracle over keys 0..r. (Wider scores would carry the f32 rounding
    # of the dot products, about 1e-6 of a score here, past the f32 bar.)
    pa, lib, stream, enc = env
    S = 2048
    q = 1.5 * O.normal(91 + Hd, (1, Nq, S, Hd))
    k = 1.5 * O.normal(92 + Hd, (1, Nkv, S, Hd))
    v = O.normal(93 + Hd, (1, Nkv, S, Hd))
    scale = 2 / np.sqrt(Hd)
    to = upload(pa, np.full((1, Nq, S, Hd), np.nan, np.float32), "f32")
    kern = pa.Kernels.FlashAttention(upload(pa, q, "f32"), upload(pa, k, "f32"), upload(pa, v, "f32"), out=to,
                                     scale=scale, batch=1, query_heads=Nq, kv_heads=Nkv, query_len=S, key_len=S,
                                     head_dim=Hd)
    assert kern.function_names == [f"flash_attention_tiled16_f32_f32_d{Hd}"]
    enc.encode(kern)
    stream.synchronize()
    got = download(to, stream).reshape(1, Nq, S, Hd)
    assert not np.isnan(got).any()
    for r in (0, 15, 16, 127, 1000, 2047):
        ref = O.attention_naive(q[:, :, r:r + 1], k[:, :, :r + 1].copy(), v[:, :, :r + 1].copy(), scale)
        assert_out(got[:, :, r:r + 1], ref, EPS["f32"], "f32", f"f32 Hd {Hd} row {r}")


@pytest.mark.parametrize("dtype,Hd", [("f16", 64), ("bf16", 128), ("f16", 256), ("bf16", 512), ("f32", 128),
                                      ("f32", 512)])
def test_tiled_attention_ignores_cache_past_key_len(env, rows, dtype, Hd):
    # K/V rows past key_len in a larger cache are not keys: here they hold
    # NaN (a cache is filled only up to the current length), and the last
    # key step, ragged (Sk = 100), reaches into them
    pa, lib, stream, enc = env
    B, Nq, Nkv, Sq, Sk, cap = 1, 2, 1, 70, 100, 160
    q = rounded(O.normal(31 + Hd, (B, Nq, Sq, Hd)), dtype)
    k = rounded(O.normal(32 + Hd, (B, Nkv, cap, Hd)), dtype)
    v = rounded(O.normal(33 + Hd, (B, Nkv, cap, Hd)), dtype)
    k[:, :, Sk:] = np.nan
    v[:, :, Sk:] = np.nan
    scale = 1 / np.sqrt(Hd)
    to = pa.Tensor.empty([B, Nq, Sq, Hd], dtype)
    kern = pa.Kernels.FlashAttention(upload(pa, q, dtype), upload(pa, k, dtype), upload(pa, v, dtype), out=to,
                                     scale=scale, batch=B, query_heads=Nq, kv_heads=Nkv, query_len=Sq, key_len=Sk,
                                     head_dim=Hd, key_capacity=cap)
    assert kern.function_names[0].startswith("flash_attention_tiled")
    enc.encode(kern)
    stream.synchronize()
    got = download(to, stream).reshape(B, Nq, Sq, Hd)
    assert not np.isnan(got).any(), "a key past key_len entered the output"
    ref = O.attention_naive(q, k, v, scale, key_len=Sk)
    assert_out(got, ref, EPS[dtype], dtype, f"cache past key_len {dtype} Hd {Hd}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_tiled_attention_hd512_sampled(env, dtype):
    # a Gemma-4-shaped global-attention prefill: [1, 8, 2048, 512], GQA 2:1,
    # causal, scale 1/sqrt(512): 32 tiles of 64 rows per head. Sampled query
    # rows against the oracle over keys 0..r, from a NaN-filled output.
    pa, lib, stream, enc = env
    Nq, Nkv, S, Hd = 8, 4, 2048, 512
    tq = pa.Tensor.empty([1, Nq, S, Hd], dtype)
    tk, tv = (pa.Tensor.empty([1, Nkv, S, Hd], dtype) for _ in range(2))
    for i, t in enumerate((tq, tk, tv)):
        lib.fill_normal(t, 50 + i, stream=stream)
    to = upload(pa, np.full((1, Nq, S, Hd), np.nan, np.float32), dtype)
    scale = 1 / np.sqrt(Hd)
    kern = pa.Kernels.FlashAttention(tq, tk, tv, out=to, scale=scale, batch=1, query_heads=Nq, kv_heads=Nkv,
                                     query_len=S, key_len=S, head_dim=Hd)
    assert kern.function_names == [f"flash_attention_tiled16_{dtype}_{dtype}_d512"]
    enc.encode(kern)
    stream.synchronize()
    q = download(tq, stream).reshape(1, Nq, S, Hd)
    k, v = (download(t, stream).reshape(1, Nkv, S, Hd) for t in (tk, tv))
    got = download(to, stream).reshape(1, Nq, S, Hd)
    assert not np.isnan(got).any()
    for r in (0, 63, 64, 1000, 2047):
        ref = O.attention_naive(q[:, :, r:r + 1], k[:, :, :r + 1].copy(), v[:, :, :r + 1].copy(), scale)
        assert_out(got[:, :, r:r + 1], ref, EPS[dtype], dtype, f"Hd 512 {dtype} row {r}")


@pytest.mark.parametrize("dtype,ot", [("f16", "f16"), ("bf16", "bf16"), ("bf16", "f32")])
@pytest.mark.parametrize("B,Nq,Nkv,Sq,Sk,Hd", [
    (1, 2, 1, 512, 512, 64),
    (2, 2, 1, 520, 700, 128),   # Sq < Sk, ragged last tile: every tile split
    (1, 2, 2, 640, 640, 256),
])
def test_tiled_attention_split_tiles_vs_oracle(env, rows, dtype, ot, B, Nq, Nkv, Sq, Sk, Hd):
    # causal prefill with few tiles per CU: light and heavy query tiles
    # paired into blocks of equal work, the heavy tile of a pair split over
    # the two blocks and its parts merged by the pair's second block
    pa = env[0]
    q = rounded(O.normal(Sq + Hd + 7, (B, Nq, Sq, Hd)), dtype)
    k = rounded(O.normal(Sk + Hd + 8, (B, Nkv, Sk, Hd)), dtype)
    v = rounded(O.normal(Sk + Hd + 9, (B, Nkv, Sk, Hd)), dtype)
    scale = 1 / np.sqrt(Hd)
    got, kern = _attend(env, q, k, v, dtype, ot, scale, pa.AttentionMask(0, -1))
    assert kern.function_names == _paired(dtype, ot, Hd, rows)
    ref = O.attention_naive(q, k, v, scale, mask_kind=0)
    assert not np.isnan(got).any()
    assert_out(got, ref, EPS[dtype], ot, f"split tiled attention {dtype}->{ot} Sq={Sq} Sk={Sk} Hd={Hd}")


@pytest.mark.parametrize("Hd", [64, 256])
def test_tiled_attention_pairs_with_merge_kernel(env, monkeypatch, Hd):
    # POPCORN_FA_PAIR_MERGE=0: paired tiles merged by the split-merge kernel
    # (pairTiles 1) instead of the pair's second block
    monkeypatch.setenv("POPCORN_FA_PAIR_MERGE", "0")
    pa = env[0]
    B, Nq, Nkv, S, dtype = 1, 2, 1, 640, "f16"
    q = rounded(O.normal(S + Hd + 1, (B, Nq, S, Hd)), dtype)
    k = rounded(O.normal(S + Hd + 2, (B, Nkv, S, Hd)), dtype)
    v = rounded(O.normal(S + Hd + 3, (B, Nkv, S, Hd)), dtype)
    scale = 1 / np.sqrt(Hd)
    got, kern = _attend(env, q, k, v, dtype, dtype, scale, pa.AttentionMask(0, -1))
    assert kern.function_names[1] == f"flash_attention_split_merge_{dtype}_d{Hd}"
    ref = O.attention_naive(q, k, v, scale, mask_kind=0)
    assert_out(got, ref, EPS[dtype], dtype, f"paired tiles, merge kernel, Hd={Hd}")


@pytest.mark.parametrize("Hd", [64, 256])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_tiled_attention_wide_score_range(env, rows, dtype, Hd):
    # scores spread over hundreds of natural-log units (scale 1, inputs x 3):
    # the running max moves often and far, so the lazy rescale (the reference
    # max moves only when a score passes it by more than 8) is exercised on
    # most steps, split tiles included
    pa = env[0]
    B, Nq, Nkv, S = 1, 2, 1, 640
    q = rounded(3.0 * O.normal(901, (B, Nq, S, Hd)), dtype)
    k = rounded(3.0 * O.normal(902, (B, Nkv, S, Hd)), dtype)
    v = rounded(O.normal(903, (B, Nkv, S, Hd)), dtype)
    got, kern = _attend(env, q, k, v, dtype, dtype, 1.0, pa.AttentionMask(0, -1))
    assert kern.function_names[0] == _tiled(dtype, dtype, Hd, rows)
    ref = O.attention_naive(q, k, v, 1.0, mask_kind=0)
    assert np.isfinite(got).all()
    assert_out(got, ref, EPS[dtype], dtype, f"wide-range tiled attention {dtype}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_tiled_attention_config5_sampled(env, rows, dtype):
    # BASELINE config 5 attention: [1, 16, 2048, 256] f16 (and bf16), causal,
    # scale 1/16. A sampled query row r is checked as a single-row query over
    # keys 0..r (the same posQ = r), against the oracle; the output starts as
    # NaN, so a row either kernel skips fails.
    pa, lib, stream, enc = env
    H, S, Hd = 16, 2048, 256
    tq, tk, tv = (pa.Tensor.empty([1, H, S, Hd], dtype) for _ in range(3))
    for i, t in enumerate((tq, tk, tv)):
        lib.fill_normal(t, 40 + i, stream=stream)
    to = upload(pa, np.full((1, H, S, Hd), np.nan, np.float32), dtype)
    kern = pa.Kernels.FlashAttention(tq, tk, tv, out=to, scale=1 / 16, batch=1, query_heads=H, kv_heads=H,
                                     query_len=S, key_len=S, head_dim=Hd)
    # 16 tiles per head on 256 CUs: light and heavy tiles paired, the heavy ones split
    assert kern.function_names == _paired(dtype, dtype, Hd, rows)
    # twice: the second launch finds the ready flags the first one reset
    for rep in range(2):
        if rep:
            lib.fill_normal(tq, 60, stream=stream)
            to.copy_from(O.to_bits(np.full((1, H, S, Hd), np.nan, np.float32), TAG[dtype]), stream)
        enc.encode(kern)
        stream.synchronize()
        q, k, v = (download(t, stream).reshape(1, H, S, Hd) for t in (tq, tk, tv))
        got = download(to, stream).reshape(1, H, S, Hd)
        assert not np.isnan(got).any()
        for r in (0, 1, 127, 128, 1000, 1151, 1152, 2047):
            ref = O.attention_naive(q[:, :, r:r + 1], k[:, :, :r + 1].copy(), v[:, :, :r + 1].copy(), 1 / 16)
            assert_out(got[:, :, r:r + 1], ref, EPS[dtype], dtype, f"config5 {dtype} launch {rep} row {r}")


def test_tiled_attention_two_tiles_per_cu_sampled(env, rows):
    # 24 heads x 16 tiles on 256 CUs (up to two tiles per CU): the tiles
    # with more than half the last tile's key steps run as two blocks over
    # the halves of their keys, merged by the merge kernel (f16, Hd 256,
    # causal). Sampled rows as in the config-5 test, from a NaN-filled output.
    pa, lib, stream, enc = env
    H, S, Hd = 24, 2048, 256
    tq, tk, tv = (pa.Tensor.empty([1, H, S, Hd], "f16") for _ in range(3))
    for i, t in enumerate((tq, tk, tv)):
        lib.fill_normal(t, 70 + i, stream=stream)
    to = upload(pa, np.full((1, H, S, Hd), np.nan, np.float32), "f16")
    kern = pa.Kernels.FlashAttention(tq, tk, tv, out=to, scale=1 / 16, batch=1, query_heads=H, kv_heads=H,
                                     query_len=S, key_len=S, head_dim=Hd)
    assert kern.function_names == [_tiled("f16", "f16", Hd, rows), "flash_attention_split_merge_f16_d256"]
    enc.encode(kern)
    stream.synchronize()
    q, k, v = (download(t, stream).reshape(1, H, S, Hd) for t in (tq, tk, tv))
    got = download(to, stream).reshape(1, H, S, Hd)
    assert not np.isnan(got).any()
    for r in (0, 127, 1023, 1024, 1100, 1535, 2047):
        ref = O.attention_naive(q[:, :, r:r + 1], k[:, :, :r + 1].copy(), v[:, :, :r + 1].copy(), 1 / 16)
        assert_out(got[:, :, r:r + 1], ref, EPS["f16"], "f16", f"two tiles per CU row {r}")


def _merged_pair_launch(pa, lib, stream, tq, tk, tv, out, pO, pML, flags, B, Nq, S, Hd, dtype, ticket):
    """A raw launch of the 16-row kernel with pairTiles 2 (causal)."""
    import struct
    nQT = (S + 127) // 128
    nSplit = nQT // 2
    # TiledFlashAttentionConstants: B, Nq, Nkv, Sq, Sk, Hd, qTilesPerHead,
    # maskKind (0: causal), slidingWindow (-1), scale, kvStride, splitFrom,
    # pairTiles, ticketLo, ticketHi
    consts = struct.pack("<8Iif5I", B, Nq, Nq, S, S, Hd, nQT, 0, -1, 1 / np.sqrt(Hd), 0,
                         nQT - nSplit, 2, ticket & 0xFFFFFFFF, ticket >> 32)
    lib.launch(f"flash_attention_tiled16_{dtype}_{dtype}_d{Hd}", (B * Nq * nQT, 1, 1), (512, 1, 1),
               [tq.ptr, tk.ptr, tv.ptr, out.ptr, pO.ptr, pML.ptr, flags.ptr], [consts], stream=stream)


def _pair_buffers(pa, tiles, Hd, stream):
    """The exchange of a raw merged-pair launch, in uncached memory as the
    kernel requires: pO, pML and the flags (abort word + one per tile), zeroed."""
    pO = pa.Tensor.empty_uncached([tiles * 128, Hd], "f32")
    pML = pa.Tensor.empty_uncached([tiles * 128 * 2], "f32")
    flags = pa.Tensor.empty_uncached([1 + tiles], "u64")
    flags.copy_from(np.zeros(1 + tiles, np.uint64), stream)
    return pO, pML, flags


def test_merged_pairs_reset_ready_flags(env):
    # A raw launch of the 16-row kernel with pairTiles 2 (causal, 2 heads x 5
    # tiles: two pairs and a middle tile per head) twice with the same
    # ticket, as a replayed graph would: after each launch every ready flag
    # and the abort word are 0 (the merging block resets its flag), and the
    # second launch, over new queries, matches the oracle too.
    pa, lib, stream, enc = env
    B, Nq, S, Hd, dtype = 1, 2, 640, 128, "f16"
    tiles = B * Nq * (((S + 127) // 128) // 2)
    ticket = 0x5EED1234ABCD0001
    k = rounded(O.normal(11, (B, Nq, S, Hd)), dtype)
    v = rounded(O.normal(12, (B, Nq, S, Hd)), dtype)
    tk, tv = upload(pa, k, dtype), upload(pa, v, dtype)
    pO, pML, flags = _pair_buffers(pa, tiles, Hd, stream)
    for rep in range(2):
        q = rounded(O.normal(20 + rep, (B, Nq, S, Hd)), dtype)
        tq = upload(pa, q, dtype)
        out = upload(pa, np.full((B, Nq, S, Hd), np.nan, np.float32), dtype)
        _merged_pair_launch(pa, lib, stream, tq, tk, tv, out, pO, pML, flags, B, Nq, S, Hd, dtype, ticket)
        stream.synchronize()
        f = flags.numpy(stream)
        assert (f == 0).all(), f"launch {rep}: ready flags or abort word not reset: {f}"
        got = download(out, stream).reshape(B, Nq, S, Hd)
        ref = O.attention_naive(q, k, v, 1 / np.sqrt(Hd), mask_kind=0)
        assert_out(got, ref, EPS[dtype], dtype, f"merged pairs, launch {rep}")


def test_merged_pairs_give_up_is_replay_safe(env):
    # The give-up path, forced from the host: split tile 1 (head 0, query
    # tile 4: rows 512..639) starts with its flag poisoned, as a merging
    # block that gave up leaves it. Its merging block must not wait or merge:
    # it writes NaN rows and sets the abort word, and its publishing block's
    # compare-and-swap from 0 leaves the poison in place. A second launch
    # with the same ticket (a replayed graph) fails the same way instead of
    # taking a stale part. Every other tile matches the oracle. Once the
    # flags are cleared, a third launch is whole.
    pa, lib, stream, enc = env
    B, Nq, S, Hd, dtype = 1, 2, 640, 128, "f16"
    tiles = B * Nq * (((S + 127) // 128) // 2)
    ticket = 0x0123456789ABCDEF
    poison = np.uint64(0xFFFFFFFFFFFFFFFF)
    q = rounded(O.normal(31, (B, Nq, S, Hd)), dtype)
    k = rounded(O.normal(32, (B, Nq, S, Hd)), dtype)
    v = rounded(O.normal(33, (B, Nq, S, Hd)), dtype)
    tq, tk, tv = upload(pa, q, dtype), upload(pa, k, dtype), upload(pa, v, dtype)
    ref = O.attention_naive(q, k, v, 1 / np.sqrt(Hd), mask_kind=0)
    pO, pML, flags = _pair_buffers(pa, tiles, Hd, stream)
    init = np.zeros(1 + tiles, np.uint64)
    init[1 + 1] = poison
    flags.copy_from(init, stream)
    bad = np.zeros((B, Nq, S), bool)
    bad[0, 0, 512:640] = True
    for rep in range(3):
        if rep == 2:
            flags.copy_from(np.zeros(1 + tiles, np.uint64), stream)
        out = upload(pa, np.full((B, Nq, S, Hd), 7.0, np.float32), dtype)
        _merged_pair_launch(pa, lib, stream, tq, tk, tv, out, pO, pML, flags, B, Nq, S, Hd, dtype, ticket)
        stream.synchronize()
        f = flags.numpy(stream)
        got = download(out, stream).reshape(B, Nq, S, Hd)
        if rep < 2:
            assert f[0] == 1, f"launch {rep}: abort word not set"
            assert f[2] == poison, f"launch {rep}: the poisoned flag was overwritten: {f[2]:#x}"
            assert (np.delete(f, [0, 2]) == 0).all(), f
            assert np.isnan(got[bad]).all(), f"launch {rep}: the given-up tile's rows are not NaN"
            assert not np.isnan(got[~bad]).any()
            assert_out(got[~bad], ref[~bad], EPS[dtype], dtype, f"merged pairs around a given-up tile, launch {rep}")
        else:
            assert (f == 0).all(), f
            assert_out(got, ref, EPS[dtype], dtype, "merged pairs after the flags were cleared")


def test_merged_pairs_abort_reported_at_stream_sync(env):
    # The stream's own exchange (the descriptor path): a poisoned flag makes
    # the launch write NaN rows for that tile, and popcorn_stream_synchronize
    # reports -1019 and clears the flags; the next launch is whole.
    pa, lib, stream, enc = env
    B, Nq, S, Hd, dtype = 1, 2, 640, 128, "f16"
    q = rounded(O.normal(41, (B, Nq, S, Hd)), dtype)
    k = rounded(O.normal(42, (B, Nq, S, Hd)), dtype)
    v = rounded(O.normal(43, (B, Nq, S, Hd)), dtype)
    ref = O.attention_naive(q, k, v, 1 / np.sqrt(Hd), mask_kind=0)
    tq, tk, tv = upload(pa, q, dtype), upload(pa, k, dtype), upload(pa, v, dtype)
    to = pa.Tensor.empty([B, Nq, S, Hd], dtype)
    kern = pa.Kernels.FlashAttention(tq, tk, tv, out=to, scale=1 / np.sqrt(Hd), batch=B, query_heads=Nq,
                                     kv_heads=Nq, query_len=S, key_len=S, head_dim=Hd)
    assert kern.function_names == [f"flash_attention_tiled16_{dtype}_{dtype}_d{Hd}"]
    stream.synchronize()
    flags = pa.attention_pair_flags(stream)
    init = np.zeros(flags.shape[0], np.uint64)
    init[1 + 3] = np.uint64(0xFFFFFFFFFFFFFFFF)  # split tile 3: head 1, query tile 4
    flags.copy_from(init, stream)
    enc.encode(kern)
    with pytest.raises(pa.PopcornError) as e:
        stream.synchronize()
    assert e.value.code == pa.PopcornError.GPU_INTERNAL
    got = download(to, stream).reshape(B, Nq, S, Hd)
    assert np.isnan(got[0, 1, 512:640]).all() and not np.isnan(got[0, 0]).any()
    assert (flags.numpy(stream) == 0).all()
    enc.encode(kern)
    stream.synchronize()
    assert_out(download(to, stream).reshape(B, Nq, S, Hd), ref, EPS[dtype], dtype, "merged pairs after the abort")


def test_merged_pairs_bitwise_stable_over_launches(env):
    # Config-5 attention (f16, 16 heads x 2048, Hd 256, causal: merged pairs)
    # launched 200 times, with a split-K GEMM borrowing and writing pooled
    # scratch between launches; every output must equal the first bit for
    # bit (the merge is deterministic), stopping at the first difference.
    pa, lib, stream, enc = env
    H, S, Hd = 16, 2048, 256
    tq, tk, tv = (pa.Tensor.empty([1, H, S, Hd], "f16") for _ in range(3))
    for i, t in enumerate((tq, tk, tv)):
        lib.fill_normal(t, 80 + i, stream=stream)
    to = pa.Tensor.empty([1, H, S, Hd], "f16")
    kern = pa.Kernels.FlashAttention(tq, tk, tv, out=to, scale=1 / 16, batch=1, query_heads=H, kv_heads=H,
                                     query_len=S, key_len=S, head_dim=Hd)
    assert kern.function_names == [_tiled("f16", "f16", Hd, "rows16")]
    # a down-projection-shaped split-K GEMM: its f32 partials in pooled scratch
    ga, gb = pa.Tensor.empty([1024, 24576], "f16"), pa.Tensor.empty([3072, 24576], "f16")
    lib.fill_normal(ga, 90, stream=stream)
    lib.fill_normal(gb, 91, std=0.02, stream=stream)
    gc = pa.Tensor.empty([1024, 3072], "f16")
    gemm = pa.Kernels.Matmul(ga, gb, gc, True)
    assert gemm.function_names[1] == "matmul_splitk_reduce_f16"
    first = None
    for i in range(200):
        enc.encode(kern)
        enc.encode(gemm)
        stream.synchronize()
        got = to.numpy(stream)
        if first is None:
            first = got
            assert not np.isnan(first.view(np.float16)).any()
        elif not np.array_equal(got, first):
            diff = int(np.count_nonzero(got != first))
            raise AssertionError(f"launch {i}: {diff} output elements differ from the first launch")
