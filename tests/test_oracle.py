"""Pins the CPU oracle before it is trusted as the checker.

Each test checks an oracle function against something other than its own
formula: a known-answer test from the reference's test suite (cited), an
independent implementation (numpy float64 / float16, torch bfloat16), a
closed form, or brute force on a tiny input.
"""
import json
import os

import numpy as np
import pytest

from conftest import assert_approx

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---- generators --------------------------------------------------------------

def test_xorshift_matches_golden(oracle):
    with open(os.path.join(GOLDEN, "xorshift64.json")) as f:
        g = json.load(f)
    got = oracle.xorshift64_sequence(int(g["seed"], 16), len(g["outputs"]))
    assert [f"{int(v):016x}" for v in got] == g["outputs"]
    fl = oracle.fa_test_floats(int(g["seed"], 16), len(g["fa_test_floats"]))
    np.testing.assert_array_equal(fl, np.array(g["fa_test_floats"], dtype=np.float32))


def test_fa_test_floats_range(oracle):
    x = oracle.fa_test_floats(0xDEADBEEFCAFEBABE, 20000)
    assert np.all(np.abs(x) <= 0.2 + 1e-7)
    assert abs(x.mean()) < 0.01 and 0.10 < x.std() < 0.13  # uniform(-.2,.2): std .1155


def test_normal_moments(oracle):
    z = oracle.normal(0, (400000,))
    assert abs(z.mean()) < 0.01
    assert abs(z.std() - 1.0) < 0.01
    # tail fractions of N(0,1): P(|z|>1)=.3173, P(|z|>2)=.0455
    assert abs(np.mean(np.abs(z) > 1) - 0.3173) < 0.005
    assert abs(np.mean(np.abs(z) > 2) - 0.0455) < 0.002
    w = oracle.normal(3, (1000,), mean=1.0, std=0.1)
    assert abs(w.mean() - 1.0) < 0.02
    assert not np.array_equal(oracle.normal(0, (16,)), oracle.normal(1, (16,)))
    np.testing.assert_array_equal(oracle.normal(5, (33,)), oracle.normal(5, (33,)))


# ---- conversions ------------------------------------------------------------

def test_bf16_store_formula_special_cases(oracle):
    def bf(bits):  # through memory, so signalling NaNs are not quieted on the way
        x = np.array([bits], np.uint32).view(np.float32)
        return int(oracle.to_bits(x, oracle.BF16)[0])

    assert bf(0x3F808000) == 0x3F80  # tie, even stays
    assert bf(0x3F818000) == 0x3F82  # tie, odd rounds up
    assert bf(0x3F808001) == 0x3F81
    # PopcornDTypes.h:29-34 has no NaN case: this NaN rounds to +Inf
    assert bf(0x7F800001) == 0x7F80
    assert bf(0x7F7FFFFF) == 0x7F80  # rounds up to inf
    assert bf(0xFFC00000) == 0xFFC0  # quiet NaN stays NaN
    assert oracle.from_bits(np.array([0x3F80], np.uint16), oracle.BF16)[0] == 1.0


def test_bf16_matches_torch_rne(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    ours = oracle.to_bits(x, oracle.BF16)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    # torch gives inf for overflow as well; the formula agrees on every finite input
    np.testing.assert_array_equal(ours, ref)


def test_f16_matches_numpy(oracle):
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2.0**-24, 2.0**-25,
                        3 * 2.0**-26, 2.0**-14, np.inf, -np.inf, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11],
                       np.float32)
    scaled = (rng.standard_normal(100000) * np.exp(rng.uniform(-25, 12, 100000))).astype(np.float32)
    for arr in (x[np.isfinite(x)], special, scaled):
        ours = oracle.to_bits(arr, oracle.F16)
        ref = arr.astype(np.float16).view(np.uint16)
        np.testing.assert_array_equal(ours, ref)
    nan = oracle.to_bits(np.array([np.nan], np.float32), oracle.F16)
    assert (nan[0] & 0x7C00) == 0x7C00 and (nan[0] & 0x3FF) != 0
    h = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    back = oracle.from_bits(h, oracle.F16)
    ref = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    np.testing.assert_array_equal(back[finite], ref[finite])
    assert np.all(np.isnan(back[np.isnan(ref)]))


# ---- KV-cache write ---------------------------------------------------------

def test_kv_cache_write_reference_kat(oracle):
    # Tests/PopcornTests/Kernels/KernelsTests.swift:551-564
    src = np.array([1, 2, 3, 4], np.float32).reshape(1, 1, 2, 2)
    cache = np.zeros((1, 1, 4, 2), np.float32)
    assert oracle.kv_cache_write(src, oracle.F32, cache, oracle.F32, offset=1) == 0
    assert cache.ravel().tolist() == [0, 0, 1, 2, 3, 4, 0, 0]


def test_kv_cache_write_bf16_paths(oracle):
    rng = np.random.default_rng(3)
    src = rng.standard_normal((2, 3, 5, 7)).astype(np.float32)
    # f32 -> bf16 uses the store formula elementwise
    cache = np.zeros((2, 3, 11, 7), np.uint16)
    assert oracle.kv_cache_write(src, oracle.F32, cache, oracle.BF16, offset=4) == 0
    np.testing.assert_array_equal(cache[:, :, 4:9], oracle.to_bits(src, oracle.BF16))
    assert not cache[:, :, :4].any() and not cache[:, :, 9:].any()
    # bf16 -> bf16 is the identity on bits, NaN payloads included
    bits = rng.integers(0, 65536, (1, 2, 3, 4), dtype=np.uint32).astype(np.uint16)
    cache = np.zeros((1, 2, 3, 4), np.uint16)
    assert oracle.kv_cache_write(bits, oracle.BF16, cache, oracle.BF16, offset=0) == 0
    np.testing.assert_array_equal(cache, bits)
    # range check of KVCacheWrite.swift:45-47
    cache = np.zeros((1, 2, 3, 4), np.uint16)
    assert oracle.kv_cache_write(bits, oracle.BF16, cache, oracle.BF16, offset=1) == -1007


# ---- RMSNorm ----------------------------------------------------------------

def test_rmsnorm_reference_kats(oracle):
    # KernelsTests.swift:142-162 (Gemma-style addOne, zero weight)
    x = np.array([1, 2, 3, 4], np.float32)
    y = oracle.rmsnorm(x, np.zeros(4, np.float32), 1e-6, add_one=True)
    assert_approx(y, x / np.sqrt(np.float32(7.5)), 1e-4, "gemma kat")
    # KernelsTests.swift:164-175 (no weight, eps 0)
    y = oracle.rmsnorm(np.array([[3, 4]], np.float32), None, 0.0)
    assert_approx(y.ravel(), np.array([3, 4]) / np.sqrt(12.5), 1e-4, "no-weight kat")


def test_rmsnorm_constant_row_closed_form(oracle):
    # a constant row c gives y = sign(c) * w / sqrt(1 + eps/c^2)
    for c in (0.5, -3.0, 20.0):
        x = np.full((2, 2304), c, np.float32)
        w = np.linspace(0.5, 1.5, 2304).astype(np.float32)
        y = oracle.rmsnorm(x, w, 1e-6)
        expect = np.sign(c) * w / np.sqrt(1 + 1e-6 / c**2)
        assert_approx(y[0], expect, 1e-5, "constant row")
        assert_approx(y[1], expect, 1e-5, "constant row 2")


def test_rmsnorm_vs_float64(oracle):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 777)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(777)).astype(np.float32)
    y = oracle.rmsnorm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64**2).mean(-1, keepdims=True) + 1e-6) * w
    assert_approx(y, ref, 1e-5, "rmsnorm f64")


# ---- Matmul -----------------------------------------------------------------

def test_matmul_reference_kats(oracle):
    a = np.array([1, 2, 3, 4, 5, 6], np.float32)
    # KernelsTests.swift:179-190
    c = oracle.matmul(a, np.array([7, 8, 9, 10, 11, 12], np.float32), 2, 3, 2, False)
    assert c.ravel().tolist() == [58, 64, 139, 154]
    # KernelsTests.swift:217-229 (transposeB)
    c = oracle.matmul(a, np.array([7, 9, 11, 8, 10, 12], np.float32), 2, 3, 2, True)
    assert c.ravel().tolist() == [58, 64, 139, 154]
    # KernelsTests.swift:192-199 (m == 1, matvec)
    c = oracle.matmul(np.array([1, 2, 3], np.float32), np.array([7, 9, 11, 8, 10, 12], np.float32), 1, 3, 2, True)
    assert c.ravel().tolist() == [58, 64]


@pytest.mark.parametrize("M,K,N,tb", [(1, 256, 67, True), (1, 131, 64, True), (64, 64, 64, False),
                                      (70, 33, 50, False), (64, 64, 64, True)])
def test_matmul_integer_exact(oracle, M, K, N, tb):
    # shapes of KernelsTests.swift:204-215 and :278-294; small integers make every
    # partial sum exact in f32, so the result must equal int64 arithmetic
    rng = np.random.default_rng(M * 1000 + K + N)
    a = rng.integers(-8, 9, (M, K))
    b = rng.integers(-8, 9, (N, K) if tb else (K, N))
    ref = a @ (b.T if tb else b)
    c = oracle.matmul(a.astype(np.float32), b.astype(np.float32), M, K, N, tb)
    np.testing.assert_array_equal(c, ref.astype(np.float32))


# ---- Elementwise ------------------------------------------------------------

def test_gelu_reference_kat(oracle):
    # KernelsTests.swift:106-117 (torch values, eps 1e-4)
    y = oracle.gelu_tanh(np.array([0, 1, -1, 2], np.float32))
    assert_approx(y, [0.0, 0.8411920, -0.1588080, 1.9545977], 1e-4, "gelu kat")


def test_gelu_vs_torch_and_clamp(oracle):
    torch = pytest.importorskip("torch")
    x = np.linspace(-12, 12, 20001).astype(np.float32)
    ref = torch.nn.functional.gelu(torch.from_numpy(x).double(), approximate="tanh").numpy()
    assert_approx(oracle.gelu_tanh(x), ref, 1e-5, "gelu grid")
    # the +-20 clamp (GeluTanh.metal:8): far tails are exactly x and 0
    big = np.array([50.0, -50.0], np.float32)
    assert oracle.gelu_tanh(big).tolist() == [50.0, -0.0]


def test_mul_add_reference_kat(oracle):
    # KernelsTests.swift:88-95
    assert oracle.mul([1, 2, 3, 4], [5, -1, 0.5, 2]).tolist() == [5, -2, 1.5, 8]
    assert oracle.add([1, 2], [3, -4]).tolist() == [4, -2]
    # KernelsTests.swift:78-84
    assert oracle.scalar_mul([1, 2, -3, 4], 2.5).tolist() == [2.5, 5.0, -7.5, 10.0]


# ---- Attention --------------------------------------------------------------

def _attention_f64(q, k, v, scale, mask_kind=0, window=-1, key_len=None):
    q, k, v = (t.astype(np.float64) for t in (q, k, v))
    B, Nq, Sq, Hd = q.shape
    Nkv = k.shape[1]
    Sk = k.shape[2] if key_len is None else key_len
    out = np.zeros_like(q)
    for b in range(B):
        for h in range(Nq):
            hk = h * Nkv // Nq
            s = q[b, h] @ k[b, hk, :Sk].T * scale
            pos_q = Sk - Sq + np.arange(Sq)[:, None]
            pos_k = np.arange(Sk)[None, :]
            allowed = np.ones_like(s, bool) if mask_kind == 2 else pos_k <= pos_q
            if mask_kind == 1:
                allowed &= (pos_q - pos_k) < window
            s = np.where(allowed, s, -np.inf)
            m = s.max(-1, keepdims=True)
            p = np.exp(s - m)
            out[b, h] = p @ v[b, hk, :Sk] / p.sum(-1, keepdims=True)
    return out


def test_attention_gqa_one_hot_kat(oracle):
    # fixture of KernelsTests.swift:510-547: Nq=2 share the one KV head
    q = np.array([1, 0, 0, 1], np.float32).reshape(1, 2, 1, 2)
    k = np.array([1, 0, 0, 1], np.float32).reshape(1, 1, 2, 2)
    v = np.array([10, 20, 30, 40], np.float32).reshape(1, 1, 2, 2)
    out = oracle.attention_naive(q, k, v, 1.0, mask_kind=2)
    e = np.exp(1.0)
    p0 = np.array([e, 1]) / (e + 1)  # head 0 scores [1, 0]
    p1 = np.array([1, e]) / (e + 1)  # head 1 scores [0, 1]
    expect = np.stack([p0 @ [[10, 20], [30, 40]], p1 @ [[10, 20], [30, 40]]])
    assert_approx(out.reshape(2, 2), expect, 1e-6, "gqa kat")
    # a very large scale makes softmax one-hot: picks V rows exactly
    out = oracle.attention_naive(q, k, v, 1000.0, mask_kind=2)
    assert out.ravel().tolist() == [10, 20, 30, 40]


@pytest.mark.parametrize("mask_kind,window", [(0, -1), (1, 5), (2, -1)])
def test_attention_naive_vs_float64(oracle, mask_kind, window):
    rng = np.random.default_rng(10 + mask_kind)
    q = rng.standard_normal((2, 4, 7, 16)).astype(np.float32)
    k = rng.standard_normal((2, 2, 19, 16)).astype(np.float32)
    v = rng.standard_normal((2, 2, 19, 16)).astype(np.float32)
    got = oracle.attention_naive(q, k, v, 0.25, mask_kind, window, key_len=13)
    ref = _attention_f64(q, k, v, 0.25, mask_kind, window, key_len=13)
    assert_approx(got, ref, 1e-5, "naive attention")


def test_reference_bidirectional_fa_case(oracle):
    # BidirectionalFATests.swift:90-150: b1 h2 sq96 hd64, q/k/v from the seeded
    # xorshift in that order, scale 1/sqrt(64); fused vs naive maxAbs < 1e-3
    total = 1 * 2 * 96 * 64
    qkv = oracle.fa_test_floats(0xDEADBEEFCAFEBABE, 3 * total)
    q, k, v = (qkv[i * total:(i + 1) * total].reshape(1, 2, 96, 64) for i in range(3))
    naive = oracle.attention_naive(q, k, v, 1 / 8, mask_kind=2)
    fused = oracle.flash_attention_rows(q, k, v, 1 / 8, mask_kind=2)
    assert np.abs(fused - naive).max() < 1e-3
    causal = oracle.flash_attention_rows(q, k, v, 1 / 8, mask_kind=0)
    assert not np.isnan(causal).any()
    assert_approx(naive, _attention_f64(q, k, v, 1 / 8, 2), 1e-5, "bidirectional vs f64")


@pytest.mark.parametrize("P", [1, 2, 3, 8, 64, 200])
def test_flash_decoding_partition_invariance(oracle, P):
    rng = np.random.default_rng(20)
    B, Nq, Nkv, cap, Hd, Sk = 2, 8, 4, 150, 32, 137
    q = rng.standard_normal((B, Nq, 1, Hd)).astype(np.float32)
    k = rng.standard_normal((B, Nkv, cap, Hd)).astype(np.float32)
    v = rng.standard_normal((B, Nkv, cap, Hd)).astype(np.float32)
    fd, po, pm, pl = oracle.flash_decoding(q, k, v, 1 / 16, P, key_len=Sk, return_partials=True)
    naive = oracle.attention_naive(q, k, v, 1 / 16, key_len=Sk)
    assert_approx(fd, naive, 1e-5, f"FD P={P}")
    per = -(-Sk // P)
    empty = [p for p in range(P) if p * per > Sk - 1]
    for p in empty:  # FlashDecoding.metal:78-87
        assert np.all(pm[:, :, p] == -np.inf) and np.all(pl[:, :, p] == 0) and not po[:, :, p].any()


def test_flash_decoding_sliding_window(oracle):
    rng = np.random.default_rng(21)
    q = rng.standard_normal((1, 4, 1, 64)).astype(np.float32)
    k = rng.standard_normal((1, 2, 300, 64)).astype(np.float32)
    v = rng.standard_normal((1, 2, 300, 64)).astype(np.float32)
    for P in (1, 8):
        fd = oracle.flash_decoding(q, k, v, 0.125, P, mask_kind=1, window=40)
        assert_approx(fd, _attention_f64(q, k, v, 0.125, 1, 40), 1e-5, "FD window")


@pytest.mark.parametrize("Bc", [1, 16, 128])
def test_flash_attention_rows_tiles(oracle, Bc):
    rng = np.random.default_rng(22)
    q = rng.standard_normal((1, 4, 33, 32)).astype(np.float32)
    k = rng.standard_normal((1, 1, 40, 32)).astype(np.float32)
    v = rng.standard_normal((1, 1, 40, 32)).astype(np.float32)
    got = oracle.flash_attention_rows(q, k, v, 0.2, Bc=Bc)
    assert_approx(got, _attention_f64(q, k, v, 0.2), 1e-5, "FA rows causal Sq!=Sk")


# ---- Gated MLP --------------------------------------------------------------

def test_gated_mlp_f32_vs_float64(oracle):
    rng = np.random.default_rng(30)
    H, F = 96, 320
    x = rng.standard_normal(H).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    wg, wu = (0.1 * rng.standard_normal((F, H))).astype(np.float32), (0.1 * rng.standard_normal((F, H))).astype(np.float32)
    wd = (0.1 * rng.standard_normal((H, F))).astype(np.float32)
    h, out = oracle.gated_mlp(x, nw, 1e-6, wg, wu, wd)
    x64 = x.astype(np.float64)
    n = x64 / np.sqrt((x64**2).mean() + 1e-6) * nw
    g, u = wg.astype(np.float64) @ n, wu.astype(np.float64) @ n
    a = 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g**3)))
    assert_approx(h, a * u, 1e-5, "h")
    assert_approx(out, wd.astype(np.float64) @ (a * u), 1e-5, "down")


def test_gated_mlp_bf16_is_composition(oracle):
    rng = np.random.default_rng(31)
    H, F = 64, 192
    BF = oracle.BF16
    x = oracle.round_to(rng.standard_normal(H), BF)
    nw = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    wg, wu, wd = (oracle.round_to(0.02 * rng.standard_normal(s), BF) for s in ((F, H), (F, H), (H, F)))
    h, out = oracle.gated_mlp(x, nw, 1e-6, wg, wu, wd, inter_tag=BF)
    n = oracle.round_to(oracle.rmsnorm(x, nw, 1e-6), BF)
    g = oracle.round_to(oracle.matmul(n, wg, 1, H, F, True).ravel(), BF)
    u = oracle.round_to(oracle.matmul(n, wu, 1, H, F, True).ravel(), BF)
    a = oracle.round_to(oracle.gelu_tanh(g), BF)
    hh = oracle.round_to(oracle.mul(a, u), BF)
    np.testing.assert_array_equal(h, hh)
    np.testing.assert_array_equal(out, oracle.matmul(hh, wd, 1, F, H, True).ravel())


# ---- RoPE and head transposes ---------------------------------------------------

def _gemma_inv_freq(hd, base=10_000.0):
    # Gemma4Workspace.swift:195-197: 1 / base^(2i/Hd), computed in double then f32
    return np.array([1 / base ** (2 * i / hd) for i in range(hd // 2)], np.float32)


def test_rope_reference_kat(oracle):
    # KernelsTests.swift:438-489 (ropeBuildAndApply), with its approxEqual eps 1e-4
    c, s = oracle.rope_build_cos_sin([0, 1], [1.0, 0.5])
    f = np.float32
    assert_approx(c.ravel(), [1, 1, np.cos(f(1)), np.cos(f(0.5))], 1e-4, "cos")
    assert_approx(s.ravel(), [0, 0, np.sin(f(1)), np.sin(f(0.5))], 1e-4, "sin")
    x = np.arange(1, 9, dtype=np.float32).reshape(1, 2, 1, 4)
    r = oracle.rope_apply(x, c, s).ravel()
    c0, s0, c1, s1 = np.cos(1.0), np.sin(1.0), np.cos(0.5), np.sin(0.5)
    assert_approx(r[:4], [1, 2, 3, 4], 1e-4, "t=0 unchanged")
    assert_approx(r[4:], [5 * c0 - 7 * s0, 6 * c1 - 8 * s1, 5 * s0 + 7 * c0, 6 * s1 + 8 * c1], 1e-4, "t=1")


def test_rope_tables_unit_circle_and_scaling(oracle):
    # cos^2 + sin^2 = scaling^2 at every angle, large positions included; the
    # t = 0 row is (scaling, 0)
    inv = _gemma_inv_freq(256)
    pos = np.array([0, 1, 7, 4096, 131071, 1 << 20], np.int32)
    for scaling in (1.0, 0.75):
        c, s = oracle.rope_build_cos_sin(pos, inv, scaling)
        np.testing.assert_allclose(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2, scaling ** 2, rtol=1e-6)
        assert np.all(c[0] == np.float32(scaling)) and np.all(s[0] == 0)
        # angle is the f32 product float(pos) * inv_freq, then cos/sin in double
        ang = (pos.astype(np.float32)[:, None] * inv[None, :]).astype(np.float64)
        np.testing.assert_allclose(c, (np.cos(ang) * scaling).astype(np.float32), atol=2e-7)


def test_rope_rotation_properties(oracle):
    # a rotation of each (x[i], x[i + Hd/2]) pair: norms are kept, rotating by
    # +p then by -p is the identity, and p1 then p2 equals p1 + p2
    rng = np.random.default_rng(3)
    Hd, T = 64, 5
    inv = _gemma_inv_freq(Hd)
    x = rng.standard_normal((2, T, 3, Hd)).astype(np.float32)
    p = np.array([0, 3, 17, 250, 1000], np.int32)
    c, s = oracle.rope_build_cos_sin(p, inv)
    y = oracle.rope_apply(x, c, s)
    h = Hd // 2
    n_x = x[..., :h].astype(np.float64) ** 2 + x[..., h:].astype(np.float64) ** 2
    n_y = y[..., :h].astype(np.float64) ** 2 + y[..., h:].astype(np.float64) ** 2
    np.testing.assert_allclose(n_y, n_x, rtol=1e-5, atol=1e-6)
    cb, sb = oracle.rope_build_cos_sin(-p, inv)
    np.testing.assert_allclose(oracle.rope_apply(y, cb, sb), x, atol=1e-5)
    p2 = np.array([1, 2, 5, 9, 30], np.int32)
    c2, s2 = oracle.rope_build_cos_sin(p2, inv)
    c3, s3 = oracle.rope_build_cos_sin(p + p2, inv)
    np.testing.assert_allclose(oracle.rope_apply(y, c2, s2), oracle.rope_apply(x, c3, s3), atol=5e-5)
    # only the first half sees -x2*sin: a quarter turn maps (x1, x2) to (-x2, x1)
    q = np.zeros((1, 1, 1, 4), np.float32)
    q[..., 0], q[..., 2] = 1.0, 2.0
    r = oracle.rope_apply(q, np.zeros((1, 2), np.float32), np.ones((1, 2), np.float32)).ravel()
    assert r.tolist() == [-2.0, 0.0, 1.0, 0.0]


@pytest.mark.parametrize("shape", [(1, 2, 3, 4), (2, 5, 1, 7), (1, 1, 6, 256), (3, 4, 2, 1)])
def test_transpose12_vs_numpy(oracle, shape):
    x = np.arange(np.prod(shape), dtype=np.float32).reshape(shape)
    y = oracle.transpose12(x)
    np.testing.assert_array_equal(y, np.transpose(x, (0, 2, 1, 3)))
    np.testing.assert_array_equal(oracle.transpose12(y), x)


# ---- block-affine 4-bit weights ---------------------------------------------------
# The reference's tests hold no quantized case; the oracle is pinned by the
# format's bit layout, float64 algebra and exact integer products.

def test_aq_unpack_bit_layout(oracle):
    # AffineQuantizationFormat.swift:27-28: value i in bits (i % 8) * 4 of word i / 8
    words = np.array([0x87654321, 0x0000000F], np.uint32)
    assert oracle.aq_unpack(words, 16).tolist() == [1, 2, 3, 4, 5, 6, 7, 8, 15, 0, 0, 0, 0, 0, 0, 0]
    from q4util import pack_q4, unpack_q4
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, (3, 64)).astype(np.uint32)
    packed = pack_q4(q)
    assert np.array_equal(unpack_q4(packed, 64), q)
    assert oracle.aq_unpack(packed[1], 64).tolist() == q[1].tolist()


@pytest.mark.parametrize("bias", [True, False])
def test_aq_matmul_vs_float64_dequantized(oracle, bias):
    from q4util import dequantize_q4, quantize_q4
    rng = np.random.default_rng(1)
    M, N, K = 3, 40, 256
    packed, s, b, q = quantize_q4(0.05 * rng.standard_normal((N, K)), bias=bias)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = oracle.aq_matmul(x, packed, s, b, N, K)
    w64 = q.astype(np.float64) * np.repeat(s, 64, 1).astype(np.float64)
    if bias:
        w64 += np.repeat(b, 64, 1)
    assert_approx(y, x.astype(np.float64) @ w64.T, 1e-5, "aq matmul")
    # the reference's fast-path algebra: sum_g s_g sum(x q) + b_g sum(x)
    xg = x.astype(np.float64).reshape(M, K // 64, 64)
    qg = q.astype(np.float64).reshape(N, K // 64, 64)
    fast = np.einsum("mgk,ngk->mng", xg, qg) * s[None].astype(np.float64)
    if bias:
        fast += xg.sum(-1)[:, None, :] * b[None].astype(np.float64)
    assert_approx(y, fast.sum(-1), 1e-5, "aq matmul identity")
    # dequantizing first (q * s + b in f32) gives the same product
    assert_approx(y, oracle.matmul(x, dequantize_q4(q, s, b), M, K, N, True).reshape(M, N), 1e-5, "dense")


def test_aq_matmul_integer_exact(oracle):
    # x small integers, s a power of two, b an integer: every product and sum is exact
    from q4util import pack_q4
    rng = np.random.default_rng(2)
    M, N, K = 2, 24, 192
    q = rng.integers(0, 16, (N, K)).astype(np.uint32)
    s = np.full((N, K // 64), 2.0, np.float32)
    b = rng.integers(-8, 8, (N, K // 64)).astype(np.float32)
    x = rng.integers(-3, 4, (M, K)).astype(np.float32)
    w = q.astype(np.int64) * 2 + np.repeat(b, 64, 1).astype(np.int64)
    y = oracle.aq_matmul(x, pack_q4(q), s, b, N, K)
    np.testing.assert_array_equal(y, (x.astype(np.int64) @ w.T).astype(np.float32))


def test_aq_embedding_gather_vs_numpy(oracle):
    from q4util import dequantize_q4, quantize_q4
    rng = np.random.default_rng(3)
    V, H = 50, 128
    packed, s, b, q = quantize_q4(rng.standard_normal((V, H)))
    ids = np.array([7, 0, 49, 7], np.int32)
    out = oracle.aq_embedding_gather(ids, packed, s, b, H)
    np.testing.assert_array_equal(out, dequantize_q4(q, s, b)[ids])


# ---- glue -------------------------------------------------------------------

def test_argmax_and_gather_kats(oracle):
    # KernelsTests.swift:121-138
    table = np.array([0, 0, 0, 0, 1, 2, 3, 4, -1, -2, -3, -4], np.float32).reshape(3, 4)
    out = oracle.embedding_gather(np.array([2, 0, 1]), table)
    assert out.ravel().tolist() == [-1, -2, -3, -4, 0, 0, 0, 0, 1, 2, 3, 4]
    # Argmax.metal:7-9: the first of equal maxima wins
    x = np.array([[1, 5, 5, 2], [-1, -1, -3, -2]], np.float32)
    assert oracle.argmax(x).tolist() == [1, 0]


@pytest.mark.parametrize("real_block", [False, True])
def test_decoder_layer_vs_float64(oracle, real_block):
    # real_block adds the per-head q/k norms, the weightless v norm and RoPE
    # (Gemma4TextInference.swift:352-371)
    rng = np.random.default_rng(40)
    H, Nq, Nkv, Hd, F, cap, pos = 64, 4, 2, 16, 128, 12, 9
    W = {
        "in_norm": 1 + 0.1 * rng.standard_normal(H), "qkv": 0.1 * rng.standard_normal(((Nq + 2 * Nkv) * Hd, H)),
        "o": 0.1 * rng.standard_normal((H, Nq * Hd)), "post_attn_norm": 1 + 0.1 * rng.standard_normal(H),
        "pre_ffn_norm": 1 + 0.1 * rng.standard_normal(H), "gate": 0.1 * rng.standard_normal((F, H)),
        "up": 0.1 * rng.standard_normal((F, H)), "down": 0.1 * rng.standard_normal((H, F)),
        "post_ffn_norm": 1 + 0.1 * rng.standard_normal(H),
    }
    if real_block:
        W["q_norm"] = 1 + 0.1 * rng.standard_normal(Hd)
        W["k_norm"] = 1 + 0.1 * rng.standard_normal(Hd)
        W["inv_freq"] = _gemma_inv_freq(Hd)
    W = {n: w.astype(np.float32) for n, w in W.items()}
    x = rng.standard_normal(H).astype(np.float32)
    kc = rng.standard_normal((Nkv, cap, Hd)).astype(np.float32)
    vc = rng.standard_normal((Nkv, cap, Hd)).astype(np.float32)
    x0, kc0, vc0 = x.copy(), kc.copy(), vc.copy()
    oracle.decoder_layer(W, x, kc, vc, pos, H=H, Nq=Nq, Nkv=Nkv, Hd=Hd, F=F, eps=1e-6, scale=0.25,
                         act_tag=oracle.F32, v_norm=real_block, rope_scaling=1.0)

    def rms(t, w=1.0):
        return t / np.sqrt((t**2).mean(axis=-1, keepdims=True) + 1e-6) * w

    def rope(t):  # rows [n, Hd]: pair (i, i + Hd/2) turned by pos * inv_freq[i]
        ang = np.float64(np.float32(pos) * W["inv_freq"])
        h = Hd // 2
        a, b = t[:, :h], t[:, h:]
        return np.concatenate([a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)], axis=1)

    W64 = {n: w.astype(np.float64) for n, w in W.items()}
    xx = x0.astype(np.float64)
    qkv = W64["qkv"] @ rms(xx, W64["in_norm"])
    qh = qkv[:Nq * Hd].reshape(Nq, Hd)
    kh = qkv[Nq * Hd:(Nq + Nkv) * Hd].reshape(Nkv, Hd)
    vh = qkv[(Nq + Nkv) * Hd:].reshape(Nkv, Hd)
    if real_block:
        qh, kh, vh = rope(rms(qh, W64["q_norm"])), rope(rms(kh, W64["k_norm"])), rms(vh)
    q = qh.reshape(1, Nq, 1, Hd)
    kc0[:, pos] = kh
    vc0[:, pos] = vh
    np.testing.assert_allclose(kc[:, :pos + 1], kc0[:, :pos + 1], rtol=1e-5, atol=1e-6)
    att = _attention_f64(q, kc0[None].astype(np.float64), vc0[None].astype(np.float64), 0.25, key_len=pos + 1)
    xx = xx + rms(W64["o"] @ att.ravel(), W64["post_attn_norm"])
    n2 = rms(xx, W64["pre_ffn_norm"])
    g, u = W64["gate"] @ n2, W64["up"] @ n2
    a = 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g**3)))
    xx = xx + rms(W64["down"] @ (a * u), W64["post_ffn_norm"])
    assert_approx(x, xx, 1e-4, "decoder layer")


def test_half_ulp_tolerance_term():
    from conftest import half_ulp

    # bf16 keeps 8 significant bits: half an ulp at 1.0 is 2^-8, at 2.27 it is 2^-7
    assert half_ulp([1.0, 2.27, 0.0], "bf16").tolist() == [2.0**-8, 2.0**-7, 0.0]
    assert half_ulp([1.0], "f16").tolist() == [2.0**-11]
    assert half_ulp([3.0], "f32").tolist() == [0.0]
    # the bound covers exactly the store rounding of an exact value
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 10
    import oracle as O
    r = O.round_to(x, O.BF16)
    assert np.all(np.abs(r.astype(np.float64) - x) <= half_ulp(np.maximum(np.abs(r), np.abs(x)), "bf16"))
