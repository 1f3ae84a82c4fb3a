"""GPU parity of raw launches built exactly as the reference builds them.

Every kernel exported under one of the reference's host names is launched
through popcorn_launch with the reference's bindings (tensors in `tensors`
order, then the constants block, KernelCommandEncoder.swift:199-204), the
reference's constants struct (PopcornKernelTypes.h field order) and the
reference's dispatch geometry (each kernel's dispatchSize, restated below
with its citation; Metal's threads-per-grid become blocks), and its output
is compared with the oracle. A launch that does not match a kernel's
parameter list is refused with -1100 before anything runs."""
import struct

import numpy as np
import pytest

import oracle as O
from conftest import assert_approx, assert_out
from gpu_util import EPS, TAG, download, gpu_env, rounded, upload
from q4util import dequantize_q4, unpack_q4

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def u32(*v):
    return struct.pack(f"<{len(v)}I", *v)


def blocks(threads, tg):
    """Metal's dispatchThreads(grid, threadsPerThreadgroup) as a block grid."""
    return tuple((t + b - 1) // b for t, b in zip(threads, tg))


def launch(env, name, tensors, consts, threads, tg):
    pa, lib, stream, enc = env
    threads = tuple(threads) + (1,) * (3 - len(threads))
    tg = tuple(tg) + (1,) * (3 - len(tg))
    lib.launch(name, blocks(threads, tg), tg, [t.ptr for t in tensors], consts, stream=stream)
    stream.synchronize()


def elementwise_threads(count):
    # GeluTanh.swift:18, Mul.swift:19, Add.swift:52, ScalarMul.swift:18
    return ((count + 3) // 4,), (256,)


def reduction_geometry(rows, n, simd=64, max_threads=1024):
    """DispatchSize.reduction (DispatchSize.swift:6-27, :64-108) for a
    pipeline with threadExecutionWidth `simd`."""
    max_w = max(simd, min(1024, max_threads) // simd * simd)
    if rows <= 4:
        g = 8 if n <= 256 else 16 if n <= 1536 else 32
    elif rows <= 16:
        g = 4 if n <= 256 else 16 if n <= 3072 else 32
    elif rows <= 64:
        g = 4 if n <= 768 else 8 if n <= 3072 else 16 if n <= 8192 else 32
    elif rows <= 256:
        g = 1 if n <= 256 else 2 if n <= 3072 else 4 if n <= 8192 else 32
    elif rows <= 512:
        g = 1 if n <= 768 else 2 if n <= 1536 else 16 if n <= 3072 else 8 if n <= 8192 else 32
    else:
        g = 2 if n <= 768 else 8 if n <= 1536 else 32 if n <= 3072 else 16
    pref = min(max_w, g * simd)
    p2 = 1
    while p2 < n:
        p2 <<= 1
    width = max(simd, min(pref, (p2 + simd - 1) // simd * simd))
    return (width * rows,), (width,)


# ---- KV-cache write --------------------------------------------------------------

def test_kv_cache_write_reference_kat(env):
    # KernelsTests.swift:551-564: src [1, 2, 3, 4], B 1, Nkv 1, Snew 2, Smax 4,
    # Hd 2, offset 1 -> cache [0, 0, 1, 2, 3, 4, 0, 0]; KVCacheWrite.swift:33-34
    pa = env[0]
    src = pa.Tensor.from_numpy(np.array([1, 2, 3, 4], np.float32))
    cache = pa.Tensor.from_numpy(np.zeros(8, np.float32))
    launch(env, "kv_cache_write", [src, cache], [u32(1, 1, 2, 4, 2, 1)], ((4 + 3) // 4,), (256,))
    assert cache.numpy(env[2]).tolist() == [0, 0, 1, 2, 3, 4, 0, 0]


@pytest.mark.parametrize("name,st,ct", [("kv_cache_write", "f32", "f32"), ("kv_cache_write_bf16", "bf16", "bf16"),
                                        ("kv_cache_write_f32_to_bf16", "f32", "bf16")])
def test_kv_cache_write_vs_oracle(env, name, st, ct):
    pa = env[0]
    B, Nkv, Snew, Smax, Hd, off = 2, 3, 5, 17, 20, 9
    src = rounded(O.normal(1, (B, Nkv, Snew, Hd)), st)
    cache0 = rounded(O.normal(2, (B, Nkv, Smax, Hd)), ct)
    tc = upload(pa, cache0, ct)
    launch(env, name, [upload(pa, src, st), tc], [u32(B, Nkv, Snew, Smax, Hd, off)],
           ((B * Nkv * Snew * Hd + 3) // 4,), (256,))
    want = O.to_bits(cache0, TAG[ct]).copy()
    assert O.kv_cache_write(O.to_bits(src, TAG[st]), TAG[st], want, TAG[ct], off) == 0
    np.testing.assert_array_equal(tc.numpy(env[2]).ravel(), want.ravel())


# ---- attention --------------------------------------------------------------------

@pytest.mark.parametrize("t", ["f32", "bf16"])
@pytest.mark.parametrize("B,Nq,Nkv,Sk,Hd,P", [(1, 8, 4, 300, 256, 8), (2, 4, 1, 129, 64, 8), (1, 2, 2, 5, 80, 8)])
def test_flash_decoding_reference_launch(env, t, B, Nq, Nkv, Sk, Hd, P):
    # FlashDecoding.swift:54-73 with P = 8 (:77): partial over grid
    # (B * 128, Nq, P) threads of 128 (:155-160), then the combine over
    # (B * 128, Nq) (:225-230); mask causal, scale 1/sqrt(Hd)
    pa, lib, stream, enc = env
    scale = 1.0 / np.sqrt(Hd)
    q = rounded(O.normal(B + Sk, (B, Nq, 1, Hd)), t)
    k = rounded(O.normal(B + Sk + 1, (B, Nkv, Sk, Hd)), t)
    v = rounded(O.normal(B + Sk + 2, (B, Nkv, Sk, Hd)), t)
    pO = pa.Tensor.empty([B, Nq, P, Hd], "f32")
    pM, pL = pa.Tensor.empty([B, Nq, P], "f32"), pa.Tensor.empty([B, Nq, P], "f32")
    out = pa.Tensor.empty([B, Nq, 1, Hd], t)
    consts = u32(B, Nq, Nkv, Sk, Hd, P, 0) + struct.pack("<if", -1, scale)
    launch(env, f"flash_decoding_partial_{t}", [upload(pa, q, t), upload(pa, k, t), upload(pa, v, t), pO, pM, pL],
           [consts], (B * 128, Nq, P), (128,))
    launch(env, f"flash_decoding_reduce_{t}", [pO, pM, pL, out], [u32(B, Nq, Hd, P)], (B * 128, Nq, 1), (128,))
    ref = O.attention_naive(q, k, v, scale)
    assert_out(download(out, stream), ref, EPS[t], t, f"raw FlashDecoding {t}")
    # the partial maxima are the oracle's split for the same P (-inf for the
    # empty partitions when Sk < P)
    _, _, rM, _ = O.flash_decoding(q, k, v, scale, P, return_partials=True)
    gm = download(pM, stream).ravel()
    np.testing.assert_array_equal(np.isneginf(gm), np.isneginf(rM.ravel()))
    fin = np.isfinite(rM.ravel())
    assert_approx(gm[fin], rM.ravel()[fin], EPS[t], "partial m")


@pytest.mark.parametrize("name,qt,kt,ot", [("flash_attention", "f32", "f32", "f32"),
                                            ("flash_attention_bf16", "bf16", "bf16", "bf16"),
                                            ("flash_attention_bf16_to_f32", "bf16", "bf16", "f32"),
                                            ("flash_attention_f32_bf16_to_bf16", "f32", "bf16", "bf16")])
@pytest.mark.parametrize("mask,window", [(0, -1), (1, 7), (2, -1)])
def test_plain_flash_attention_reference_launch(env, name, qt, kt, ot, mask, window):
    # FlashAttention.swift:160-232: grid (B * 128, Nq, Sq) threads of 128 (:203,
    # :220-222); FlashAttentionConstants (PopcornKernelTypes.h:121-131)
    pa, lib, stream, enc = env
    B, Nq, Nkv, Sq, Sk, Hd = 2, 4, 2, 6, 45, 64
    scale = 0.125
    q = rounded(O.normal(11, (B, Nq, Sq, Hd)), qt)
    k = rounded(O.normal(12, (B, Nkv, Sk, Hd)), kt)
    v = rounded(O.normal(13, (B, Nkv, Sk, Hd)), kt)
    out = pa.Tensor.empty([B, Nq, Sq, Hd], ot)
    consts = u32(B, Nq, Nkv, Sq, Sk, Hd, mask) + struct.pack("<if", window, scale)
    launch(env, name, [upload(pa, q, qt), upload(pa, k, kt), upload(pa, v, kt), out], [consts], (B * 128, Nq, Sq), (128,))
    ref = O.attention_naive(q, k, v, scale, mask_kind=mask, window=window)
    eps = 1e-5 if (qt, kt, ot) == ("f32", "f32", "f32") else 2e-3
    assert_out(download(out, stream), ref, eps, ot, f"raw {name} mask {mask}")


# ---- matvec / matmul ------------------------------------------------------------------

@pytest.mark.parametrize("name,xt,wt,ot", [("matvec_nk_simd_f32_f32_f32", "f32", "f32", "f32"),
                                            ("matvec_nk_simd_f32_bf16_f32", "f32", "bf16", "f32"),
                                            ("matvec_nk_simd_bf16_bf16_f32", "bf16", "bf16", "f32"),
                                            ("matvec_nk_simd_bf16_bf16_bf16", "bf16", "bf16", "bf16")])
@pytest.mark.parametrize("K,N", [(256, 67), (131, 64), (2304, 9216)])
def test_matvec_nk_simd_reference_launch(env, name, xt, wt, ot, K, N):
    # Matmul.swift:246-251: threads ceil(N / 4) * 32 in threadgroups of 128;
    # shapes of KernelsTests.swift:204-215 and the Gemma gate projection
    pa, lib, stream, enc = env
    x = rounded(O.normal(K, (1, K)), xt)
    w = rounded(O.normal(K + N, (N, K), std=0.02), wt)
    out = pa.Tensor.empty([1, N], ot)
    launch(env, name, [upload(pa, x, xt), upload(pa, w, wt), out], [u32(K, N, 1)], (((N + 3) // 4) * 32,), (128,))
    ref = O.matmul(x, w, 1, K, N, True)
    assert_out(download(out, stream), ref, 1e-5 if ot == "f32" else EPS[ot], ot, f"raw {name} {K}x{N}")


@pytest.mark.parametrize("name,xt,wt,ot", [("matvec", "f32", "f32", "f32"), ("matvec_f16", "f32", "f16", "f32"),
                                            ("matvec_bf16", "f32", "bf16", "f32"),
                                            ("matvec_bf16_bf16_f32", "bf16", "bf16", "f32"),
                                            ("matvec_bf16_bf16_bf16", "bf16", "bf16", "bf16")])
def test_matvec_kn_reference_launch(env, name, xt, wt, ot):
    # Matmul.swift:268-275: one thread per output, threads N in groups of 256
    pa, lib, stream, enc = env
    K, N = 300, 517
    x = rounded(O.normal(3, (1, K)), xt)
    w = rounded(O.normal(4, (K, N), std=0.05), wt)
    out = pa.Tensor.empty([1, N], ot)
    launch(env, name, [upload(pa, x, xt), upload(pa, w, wt), out], [u32(K, N, 0)], (N,), (256,))
    assert_out(download(out, stream), O.matmul(x, w, 1, K, N, False), 1e-5 if ot == "f32" else 2e-3, ot, f"raw {name}")


@pytest.mark.parametrize("name,at,bt,ot", [("matmul", "f32", "f32", "f32"), ("matmul_f16", "f32", "f16", "f32"),
                                            ("matmul_bf16", "f32", "bf16", "f32"),
                                            ("matmul_bf16_bf16_f32", "bf16", "bf16", "f32"),
                                            ("matmul_bf16_bf16_bf16", "bf16", "bf16", "bf16")])
@pytest.mark.parametrize("tb", [False, True])
def test_matmul_reference_launch(env, name, at, bt, ot, tb):
    # Matmul.swift:62-64: threads (M, N) in 8 x 8 groups; the 2 x 3 KAT
    # (KernelsTests.swift:179-190) and 70 x 33 x 50 (:278-294)
    pa, lib, stream, enc = env
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    bb = np.ascontiguousarray(b.T) if tb else b
    c = pa.Tensor.empty([2, 2], ot)
    launch(env, name, [upload(pa, a, at), upload(pa, bb, bt), c], [u32(2, 3, 2, int(tb))], (2, 2), (8, 8))
    assert download(c, stream).ravel().tolist() == [58, 64, 139, 154]
    rng = np.random.default_rng(7)
    M, K, N = 70, 33, 50
    a = rounded(rng.uniform(-1, 1, (M, K)), at)
    b = rounded(rng.uniform(-1, 1, (N, K) if tb else (K, N)), bt)
    c = pa.Tensor.empty([M, N], ot)
    launch(env, name, [upload(pa, a, at), upload(pa, b, bt), c], [u32(M, K, N, int(tb))], (M, N), (8, 8))
    assert_out(download(c, stream), O.matmul(a, b, M, K, N, tb), 1e-5 if ot == "f32" else 2e-3, ot, f"raw {name}")


# ---- norms and elementwise ---------------------------------------------------------------

def test_rmsnorm_reference_kat(env):
    # KernelsTests.swift:142-162: [1, 2, 3, 4], weight 0 with addOne, eps 1e-6
    pa, lib, stream, enc = env
    x = pa.Tensor.from_numpy(np.array([[1, 2, 3, 4]], np.float32))
    w = pa.Tensor.from_numpy(np.zeros(4, np.float32))
    y = pa.Tensor.empty([1, 4])
    threads, tg = reduction_geometry(1, 4)
    launch(env, "rmsnorm", [x, w, y], [u32(4, 1, 1) + struct.pack("<f", 1e-6)], threads, tg)
    assert_approx(y.numpy(stream).ravel(), np.array([1, 2, 3, 4]) / np.sqrt(7.5 + 1e-6), 1e-5, "rmsnorm kat")


@pytest.mark.parametrize("name,t", [("rmsnorm", "f32"), ("rmsnorm_bf16", "bf16"), ("rmsnorm_f16", "f16")])
@pytest.mark.parametrize("rows,H", [(1, 2304), (3, 256), (70, 1000), (600, 64)])
def test_rmsnorm_reference_launch(env, name, t, rows, H):
    # RMSNorm.swift:85-86: DispatchSize.reduction(rowCount:n:) at the
    # pipeline's width (64 lanes here); f32 weight (RMSNorm.metal:42-46)
    pa, lib, stream, enc = env
    x = rounded(O.normal(rows + H, (rows, H)), t)
    w = O.normal(rows + H + 1, (H,), mean=1.0, std=0.1)
    y = pa.Tensor.empty([rows, H], t)
    threads, tg = reduction_geometry(rows, H)
    launch(env, name, [upload(pa, x, t), pa.Tensor.from_numpy(w), y], [u32(H, 1, 0) + struct.pack("<f", 1e-6)],
           threads, tg)
    assert_out(download(y, stream), O.rmsnorm(x, w, 1e-6), EPS[t], t, f"raw {name} {rows}x{H}")


@pytest.mark.parametrize("t,sfx", [("f32", ""), ("bf16", "_bf16"), ("f16", "_f16")])
def test_elementwise_reference_launch(env, t, sfx):
    pa, lib, stream, enc = env
    n = 1001
    a = rounded(O.normal(1, (n,), std=3.0), t)
    b = rounded(O.normal(2, (n,)), t)
    ta, tb = upload(pa, a, t), upload(pa, b, t)
    eps = 1e-5 if t == "f32" else 2e-3
    threads, tg = elementwise_threads(n)
    for name, ins, consts, ref in [(f"gelu_tanh{sfx}", [ta], u32(n), O.gelu_tanh(a)),
                                   (f"mul{sfx}", [ta, tb], u32(n), O.mul(a, b)),
                                   (f"add{sfx}", [ta, tb], u32(n), O.add(a, b)),
                                   (f"scalar_mul{sfx}", [ta], u32(n) + struct.pack("<f", 2.5), O.scalar_mul(a, 2.5))]:
        out = pa.Tensor.empty([n], t)
        launch(env, name, ins + [out], [consts], threads, tg)
        assert_out(download(out, stream), ref, eps, t, f"raw {name}")


# ---- RoPE, transpose, gathers ---------------------------------------------------------------

@pytest.mark.parametrize("name,xt,tt", [("rope_apply", "f32", "f32"), ("rope_apply_bf16", "bf16", "bf16"),
                                        ("rope_apply_f32_tables_bf16", "bf16", "f32")])
def test_rope_apply_reference_launch(env, name, xt, tt):
    # RopeApply.swift:37-44, :76-77: threads B * T * Nh * ceil(Hd2 / 4) in 256s
    pa, lib, stream, enc = env
    B, T, Nh, Hd = 2, 5, 3, 64
    x = rounded(O.normal(1, (B, T, Nh, Hd)), xt)
    inv = np.array([1 / 10000.0 ** (2 * i / Hd) for i in range(Hd // 2)], np.float32)
    cos, sin = O.rope_build_cos_sin(np.arange(T, dtype=np.int32) + 3, inv)
    cos, sin = rounded(cos, tt), rounded(sin, tt)
    out = pa.Tensor.empty([B, T, Nh, Hd], xt)
    launch(env, name, [upload(pa, x, xt), upload(pa, cos, tt), upload(pa, sin, tt), out], [u32(B, T, Nh, Hd // 2)],
           (B * T * Nh * ((Hd // 2 + 3) // 4),), (256,))
    assert_out(download(out, stream), O.rope_apply(x, cos, sin), 1e-5 if xt == "f32" else 2e-3, xt, f"raw {name}")


@pytest.mark.parametrize("name,t", [("transpose12", "f32"), ("transpose12_f16", "f16"), ("transpose12_bf16", "bf16")])
def test_transpose12_reference_launch(env, name, t):
    # Transpose12.swift:24, :49-50: one thread per element, groups of 256
    pa, lib, stream, enc = env
    d = (2, 3, 5, 7)
    x = rounded(O.normal(5, d), t)
    out = pa.Tensor.empty([d[0], d[2], d[1], d[3]], t)
    launch(env, name, [upload(pa, x, t), out], [u32(*d)], (int(np.prod(d)),), (256,))
    np.testing.assert_array_equal(download(out, stream), np.transpose(x, (0, 2, 1, 3)))


@pytest.mark.parametrize("name,tt,ot", [("embedding_gather", "f32", "f32"), ("embedding_gather_f16", "f16", "f16"),
                                        ("embedding_gather_bf16", "bf16", "bf16"),
                                        ("embedding_gather_bf16_to_f32", "bf16", "f32")])
def test_embedding_gather_reference_launch(env, name, tt, ot):
    # EmbeddingGather.swift:26, :117-118: threads (N, ceil(H / 4)) in (1, 64)
    pa, lib, stream, enc = env
    V, H = 50, 130
    table = rounded(O.normal(9, (V, H)), tt)
    ids = np.array([3, 0, 49, 3, 17], np.int32)
    out = pa.Tensor.empty([len(ids), H], ot)
    launch(env, name, [pa.Tensor.from_numpy(ids), upload(pa, table, tt), out], [u32(len(ids), H)],
           (len(ids), (H + 3) // 4), (1, 64))
    np.testing.assert_array_equal(download(out, stream), rounded(table[ids], ot))


def _q4(rng, N, K):
    packed = rng.integers(0, 2 ** 32, (N, K // 8), dtype=np.uint32)
    s = O.round_to(rng.uniform(0.01, 0.03, (N, K // 64)).astype(np.float32), O.BF16)
    b = O.round_to(rng.uniform(-0.2, 0.0, (N, K // 64)).astype(np.float32), O.BF16)
    return packed, s, b


@pytest.mark.parametrize("ot", ["bf16", "f32"])
def test_quantized_embedding_gather_reference_launch(env, ot):
    # EmbeddingGather.swift:90, :117-118: threads (T, H) in (1, 64)
    pa, lib, stream, enc = env
    V, H = 40, 256
    packed, s, b = _q4(np.random.default_rng(1), V, H)
    ids = np.array([5, 39, 0, 5], np.int32)
    out = pa.Tensor.empty([len(ids), H], ot)
    launch(env, f"aq_embedding_gather_bf16_{ot}_b4_g64",
           [pa.Tensor.from_numpy(ids), pa.Tensor.from_numpy(packed, "u32"), upload(pa, s, "bf16"), upload(pa, b, "bf16"),
            out], [u32(len(ids), H, H // 64, H // 8, 1)], (len(ids), H), (1, 64))
    # q * s + b in f32 (one rounding more or less than a fused multiply-add)
    assert_out(download(out, stream), O.aq_embedding_gather(ids, packed, s, b, H), 1e-6, ot, "raw aq gather",
               half_ulps=2)


@pytest.mark.parametrize("xt,ot", [("bf16", "bf16"), ("bf16", "f32"), ("f32", "f32")])
@pytest.mark.parametrize("M,N,K", [(1, 300, 2304), (3, 67, 256)])
def test_quantized_matmul_reference_launch(env, xt, ot, M, N, K):
    # Matmul.swift:311-331: aq_qmv_fast (M == 1) over M x ceil(N / 8)
    # threadgroups of 64; aq_matvec_simd4 over threads (ceil(N / 4) * 32, M)
    # in groups of min(128, max(32, ceil(N / 4) * 32))
    pa, lib, stream, enc = env
    packed, s, b = _q4(np.random.default_rng(M + N), N, K)
    x = rounded(O.normal(M * K, (M, K)), xt)
    ins = [pa.Tensor.from_numpy(packed, "u32"), upload(pa, s, "bf16"), upload(pa, b, "bf16"), upload(pa, x, xt)]
    consts = [u32(M, N, K, K // 64, K // 8, 1)]
    ref = O.aq_matmul(x, packed, s, b, N, K)
    eps = 1e-5 if xt == "f32" else 2e-3
    nb = (N + 3) // 4
    runs = [(f"aq_matvec_simd4_{xt}_bf16_{ot}_b4_g64", (nb * 32, M), (min(128, max(32, nb * 32)), 1))]
    if M == 1:
        runs.append((f"aq_qmv_fast_{xt}_bf16_{ot}_b4_g64", (M * 64, (N + 7) // 8), (64, 1)))
    for name, threads, tg in runs:
        out = pa.Tensor.empty([M, N], ot)
        launch(env, name, ins + [out], consts, threads, tg)
        if xt == "f32":
            # f32 in and out: 1e-5 of the result plus the rounding of a K-term
            # f32 sum in either order, 2e-6 of sum |x w|, against float64
            w64 = dequantize_q4(unpack_q4(packed, K), s, b).astype(np.float64)
            ref64 = x.astype(np.float64) @ w64.T
            mag = np.abs(x.astype(np.float64)) @ np.abs(w64).T
            assert (np.abs(download(out, stream) - ref64) <= 1e-5 * np.abs(ref64) + 2e-6 * mag).all(), name
        else:
            assert_out(download(out, stream), ref, eps, ot, f"raw {name}")


# ---- the launch checks ----------------------------------------------------------------------

def test_launch_not_matching_the_parameter_list_is_refused(env):
    # the extended list (3 pointers + 28 bytes) against the reference's
    # kv_cache_write_bf16 (2 + 24), and the reverse: -1100, nothing written
    pa, lib, stream, enc = env
    src = upload(pa, np.ones(8, np.float32), "bf16")
    cache0 = np.zeros(8, np.uint16)
    cache = pa.Tensor.from_numpy(cache0, "bf16")
    pos = pa.Tensor.from_numpy(np.array([0], np.int32))
    assert lib.layout("kv_cache_write_bf16") == {"buffers": 2, "constants": [24], "max_threads": 1024}
    bad = [("kv_cache_write_bf16", [src, cache, pos], [u32(1, 1, 1, 1, 8, 0, 1)]),
           ("kv_cache_write_bf16", [src, cache], [u32(1, 1, 1, 1, 8, 0, 1)]),
           ("kv_cache_write_bf16", [src, cache], [u32(1, 1, 1, 1, 8), u32(0)]),
           ("kv_cache_write_bf16_ext", [src, cache], [u32(1, 1, 1, 1, 8, 0)]),
           ("flash_decoding_partial_bf16", [src] * 7, [u32(*range(12))])]
    for name, ts, consts in bad:
        with pytest.raises(pa.PopcornError) as e:
            lib.launch(name, (1, 1, 1), (64, 1, 1), [t.ptr for t in ts], consts, stream=stream)
        assert e.value.code == pa.PopcornError.INVALID_ARGUMENT, name
        assert "parameter list" in str(e.value)
    with pytest.raises(pa.PopcornError) as e:  # block above the kernel's bound
        lib.launch("add", (1, 1, 1), (512, 1, 1), [src.ptr, src.ptr, cache.ptr], [u32(8)], stream=stream)
    assert e.value.code == pa.PopcornError.INVALID_ARGUMENT
    stream.synchronize()
    np.testing.assert_array_equal(cache.numpy(stream), cache0)


def test_custom_kernel_with_reference_bindings(env):
    # a caller-built DispatchKernel (Kernel.swift:54-70) for kv_cache_write:
    # source read, cache written, KVCacheWriteConstants; the encoder checks
    # its bindings against the kernel too
    pa, lib, stream, enc = env
    src = pa.Tensor.from_numpy(np.array([1, 2, 3, 4], np.float32))
    cache = pa.Tensor.from_numpy(np.zeros(8, np.float32))
    enc.encode(pa.Kernels.Custom("kv_cache_write", [src, cache], [1, 2], [u32(1, 1, 2, 4, 2, 1)], (1, 1, 1), (256, 1, 1)))
    stream.synchronize()
    assert cache.numpy(stream).tolist() == [0, 0, 1, 2, 3, 4, 0, 0]
    with pytest.raises(pa.PopcornError) as e:
        enc.encode(pa.Kernels.Custom("kv_cache_write", [src, cache, src], [1, 2, 1], [u32(1, 1, 2, 4, 2, 1, 0)],
                                     (1, 1, 1), (256, 1, 1)))
    assert e.value.code == pa.PopcornError.INVALID_ARGUMENT
