"""GPU parity of the block-affine 4-bit path (AffineQuantizedMatmul.metal,
AffineQuantizedEmbeddingGather.metal) against the oracle, through the C ABI:
the decode matvec (aq_qmv_fast), M > 1 rows, the any-shape kernel, and the
dequantizing gather."""
import numpy as np
import pytest

import oracle as O
from conftest import assert_out
from gpu_util import EPS, download, gpu_env, rounded, upload
import flips
from q4util import dequantize_q4, pack_q4, quantize_q4

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def _qtensor(pa, packed, s, b, N, K):
    tb = upload(pa, b, "bf16") if b is not None else None
    return pa.AffineQuantizedTensor(pa.Tensor.from_numpy(packed.view(np.uint32), "u32"), upload(pa, s, "bf16"), tb,
                                    [N, K])


def _matmul(env, x, qt, xt, ot, N, a_tensor=None):
    pa, lib, stream, enc = env
    M = x.shape[0]
    ta = a_tensor if a_tensor is not None else upload(pa, x, xt)
    tc = pa.Tensor.empty([M, N], ot)
    k = pa.Kernels.Matmul(ta, qt, tc)
    enc.encode(k)
    stream.synchronize()
    return download(tc, stream).reshape(M, N), k


@pytest.mark.parametrize("xt,ot", [("bf16", "bf16"), ("bf16", "f32"), ("f32", "f32")])
@pytest.mark.parametrize("M,N,K", [(1, 9216, 2304), (1, 2304, 9216), (1, 4096, 2304), (1, 2304, 2048),
                                   (1, 100, 64), (1, 37, 192), (3, 300, 256), (2, 64, 4160)])
@pytest.mark.parametrize("bias", [True, False])
def test_quantized_matmul_vs_oracle(env, xt, ot, M, N, K, bias):
    pa = env[0]
    rng = np.random.default_rng(N + K + M)
    packed, s, b, q = quantize_q4(0.05 * rng.standard_normal((N, K)).astype(np.float32), bias=bias)
    x = rounded(rng.standard_normal((M, K)).astype(np.float32), xt)
    got, k = _matmul(env, x, _qtensor(pa, packed, s, b, N, K), xt, ot, N)
    name = k.function_names[0]
    assert name.startswith(("aq_qmv_fast_" if M == 1 else "aq_matvec_simd4_") + f"{xt}_bf16_{ot}_b4_g64") or \
        name == f"aq_matvec_simd4_{xt}_bf16_{ot}_b4_g64"
    what = f"aq matmul {xt}->{ot} {M}x{N}x{K} bias={bias} ({name})"
    if xt == "bf16":
        # inputs exact in their dtype; f32 accumulation in another order
        assert_out(got, O.aq_matmul(x, packed, s, b, N, K), EPS[xt], ot, what)
    else:
        # f32 in and out: 1e-5 of the result plus the rounding a K-term f32 sum
        # of either order may carry, 2e-6 of sum |x w| (about 32 units in the
        # last place of that sum), against the float64 product
        w64 = dequantize_q4(q, s, b).astype(np.float64)
        ref64 = x.astype(np.float64) @ w64.T
        mag = np.abs(x.astype(np.float64)) @ np.abs(w64).T
        err = np.abs(got - ref64)
        ok = err <= 1e-5 * np.abs(ref64) + 2e-6 * mag
        assert ok.all(), f"{what}: {(~ok).sum()} elements off; max err {err.max():.3e}"
        # and the oracle (sequential f32) sits within the same bound
        ref = O.aq_matmul(x, packed, s, b, N, K)
        assert (np.abs(ref - ref64) <= 1e-5 * np.abs(ref64) + 2e-6 * mag).all()


@pytest.mark.parametrize("xt", ["bf16", "f32"])
def test_quantized_matmul_integer_exact(env, xt):
    # small integer x, scale 2, integer biases: every product and partial sum
    # is an exact f32 integer whatever the order, so the result is exact; pins
    # the nibble order and the bf16 pair staging of the fast kernel
    pa = env[0]
    rng = np.random.default_rng(9)
    N, K = 333, 2304
    q = rng.integers(0, 16, (N, K)).astype(np.uint32)
    s = np.full((N, K // 64), 2.0, np.float32)
    b = rng.integers(-8, 8, (N, K // 64)).astype(np.float32)
    x = rng.integers(-3, 4, (1, K)).astype(np.float32)
    got, k = _matmul(env, x, _qtensor(pa, pack_q4(q), s, b, N, K), xt, "f32", N)
    assert k.function_names[0].startswith("aq_qmv_fast_")
    w = q.astype(np.int64) * 2 + np.repeat(b, 64, 1).astype(np.int64)
    np.testing.assert_array_equal(got, (x.astype(np.int64) @ w.T).astype(np.float32))


def _gemm_names(ot, split=False):
    if split:
        # few tiles: the groups split over blocks, f32 partials summed once
        return ["aq_gemm_prep_bf16", "aq_gemm_mfma_bf16_bf16_splitk_b4_g64", f"matmul_splitk_reduce_{ot}"]
    return ["aq_gemm_prep_bf16", f"aq_gemm_mfma_bf16_bf16_{ot}_b4_g64"]


@pytest.mark.parametrize("ot", ["bf16", "f32"])
@pytest.mark.parametrize("M,N,K,bias,split", [(16, 16448, 1024, True, True), (100, 2700, 1024, True, True),
                                              (130, 2100, 1152, False, True), (131, 2003, 1152, True, False),
                                              (256, 1100, 2304, True, True), (300, 900, 9216, False, True),
                                              (2048, 2048, 256, True, False), (2048, 1024, 256, False, False)])
def test_quantized_gemm_vs_oracle(env, ot, M, N, K, bias, split):
    # bf16 activations with m >= 16 rows reading >= 2^27 weight bytes in all
    # take the matrix-core 4-bit GEMM (one pass over the weights for all rows; the reference runs
    # one matvec per row, Matmul.swift:279-332): group products on the matrix
    # cores, then s * D + (b - 128 s) * sum(x) per group in f32. Ragged M and
    # N (tiles of 128) included.
    pa = env[0]
    rng = np.random.default_rng(M * 7 + N + K)
    packed, s, b, q = quantize_q4(0.05 * rng.standard_normal((N, K)).astype(np.float32), bias=bias)
    x = rounded(rng.standard_normal((M, K)).astype(np.float32), "bf16")
    got, k = _matmul(env, x, _qtensor(pa, packed, s, b, N, K), "bf16", ot, N)
    # split: the tiles leave CUs idle (about two blocks per CU, at least 4
    # groups per block; 131 x 2003 is not a multiple of 4, and K 256 has too
    # few groups, so no split there)
    assert k.function_names == _gemm_names(ot, split)
    assert_out(got, O.aq_matmul(x, packed, s, b, N, K), EPS["bf16"], ot, f"aq gemm ->{ot} {M}x{N}x{K} bias={bias}")


def test_quantized_gemm_integer_exact(env):
    # small integer x, scale 2, integer biases: every product and partial sum
    # is an exact f32 integer in any order, so the GEMM's result is exact; pins
    # the nibble order, the pair order of x and both affine terms
    pa = env[0]
    rng = np.random.default_rng(19)
    M, N, K = 40, 6600, 2304
    q = rng.integers(0, 16, (N, K)).astype(np.uint32)
    s = np.full((N, K // 64), 2.0, np.float32)
    b = rng.integers(-8, 8, (N, K // 64)).astype(np.float32)
    x = rng.integers(-3, 4, (M, K)).astype(np.float32)
    got, k = _matmul(env, x, _qtensor(pa, pack_q4(q), s, b, N, K), "bf16", "f32", N)
    assert k.function_names == _gemm_names("f32", split=True)
    w = q.astype(np.int64) * 2 + np.repeat(b, 64, 1).astype(np.int64)
    np.testing.assert_array_equal(got, (x.astype(np.int64) @ w.T).astype(np.float32))


def test_quantized_gemm_threshold(env):
    # fewer than 16 rows, or under 2^27 weight bytes read in all, keep the
    # streaming matvec per row; f32 activations (held to 1e-5) never take the
    # bf16 matrix cores
    pa = env[0]
    rng = np.random.default_rng(23)
    N, K = 18000, 1024
    packed, s, b, q = quantize_q4(0.05 * rng.standard_normal((N, K)).astype(np.float32))
    qt = _qtensor(pa, packed, s, b, N, K)
    for M, xt, gemm in ((15, "bf16", False), (16, "bf16", True), (17, "f32", False)):
        x = rounded(rng.standard_normal((M, K)).astype(np.float32), xt)
        got, k = _matmul(env, x, qt, xt, "f32", N)
        assert (k.function_names[0] == "aq_gemm_prep_bf16") == gemm, (M, xt, k.function_names)
        assert_out(got, O.aq_matmul(x, packed, s, b, N, K), EPS[xt] if xt == "bf16" else 2e-5, "f32", f"M={M} {xt}")


def test_quantized_matmul_unaligned_any_kernel(env):
    # activations 2 bytes off 16-byte alignment take aq_matvec_simd4 (any shape)
    pa, lib, stream, enc = env
    rng = np.random.default_rng(4)
    N, K = 129, 320
    packed, s, b, q = quantize_q4(0.05 * rng.standard_normal((N, K)).astype(np.float32))
    x = rounded(rng.standard_normal((1, K)).astype(np.float32), "bf16")
    base = upload(pa, np.concatenate([[0.0], x.ravel()]).astype(np.float32), "bf16")
    view = pa.Tensor(base.ptr + 2, [1, K], "bf16")
    got, k = _matmul(env, x, _qtensor(pa, packed, s, b, N, K), "bf16", "bf16", N, a_tensor=view)
    assert k.function_names == ["aq_matvec_simd4_bf16_bf16_bf16_b4_g64"]
    assert_out(got, O.aq_matmul(x, packed, s, b, N, K), EPS["bf16"], "bf16", "aq any-shape")


@pytest.mark.parametrize("ot", ["bf16", "f32"])
def test_quantized_embedding_gather(env, ot):
    pa, lib, stream, enc = env
    rng = np.random.default_rng(5)
    V, H = 1000, 2304
    packed, s, b, q = quantize_q4(rng.standard_normal((V, H)).astype(np.float32))
    ids = np.array([0, 999, 17, 17, 1000, -1], np.int32)  # the last two are outside the table
    out = pa.Tensor.empty([ids.size, H], ot)
    k = pa.Kernels.EmbeddingGather(pa.Tensor.from_numpy(ids, "i32"), _qtensor(pa, packed, s, b, V, H), out)
    assert k.function_names == [f"aq_embedding_gather_bf16_{ot}_b4_g64_ext"]
    enc.encode(k)
    stream.synchronize()
    got = download(out, stream).reshape(ids.size, H)
    ref = O.aq_embedding_gather(ids[:4], packed, s, b, H)
    # q * s + b in f32 (a fused multiply-add may round once where the oracle rounds twice)
    assert_out(got[:4], ref, 1e-6, ot, "aq gather")
    assert not got[4:].any()


def _archive(path, entries):
    """A safetensors file from {name: (dtype name, shape, bytes)} in order."""
    import json
    import struct
    header, blobs, at = {}, [], 0
    for name, (dt, shape, data) in entries.items():
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [at, at + len(data)]}
        blobs.append(data)
        at += len(data)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    path.write_bytes(struct.pack("<Q", len(h)) + h + b"".join(blobs))
    return str(path)


def test_weight_loader_quantized_matmul_from_archive(env, tmp_path):
    # An MLX-style archive (Gemma4WeightLoader.swift:80-119): packed U32
    # "<name>.weight" with BF16 "<name>.scales" and "<name>.biases" -> an
    # AffineQuantizedTensor on the device; a dense BF16 weight next to it.
    from popcorn_amd.safetensors import SafeTensors, WeightLoader

    pa, lib, stream, enc = env
    rng = np.random.default_rng(8)
    N, K = 512, 2304
    packed, s, b, q = quantize_q4(0.05 * rng.standard_normal((N, K)).astype(np.float32))
    dense = rounded(0.05 * rng.standard_normal((64, K)).astype(np.float32), "bf16")
    pre = "language_model.model.layers.0.mlp."
    path = _archive(tmp_path / "q.safetensors", {
        pre + "up_proj.weight": ("U32", packed.shape, packed.tobytes()),
        pre + "up_proj.scales": ("BF16", s.shape, O.to_bits(s, O.BF16).tobytes()),
        pre + "up_proj.biases": ("BF16", b.shape, O.to_bits(b, O.BF16).tobytes()),
        pre + "down_proj.weight": ("BF16", dense.shape, O.to_bits(dense, O.BF16).tobytes()),
    })
    wl = WeightLoader(SafeTensors(path), {"bits": 4, "group_size": 64})
    assert wl.language_model_prefix == "language_model.model"
    up = wl.linear(wl.layer_prefix(0) + ".mlp.up_proj", stream)
    down = wl.linear(wl.layer_prefix(0) + ".mlp.down_proj", stream)
    assert isinstance(up, pa.AffineQuantizedTensor) and up.shape == [N, K]
    assert isinstance(down, pa.Tensor) and down.dtype == "bf16" and list(down.shape) == [64, K]
    np.testing.assert_array_equal(up.packed_values.numpy(stream), packed)
    x = rounded(rng.standard_normal((1, K)).astype(np.float32), "bf16")
    got, k = _matmul(env, x, up, "bf16", "bf16", N)
    assert k.function_names[0].startswith("aq_qmv_fast_bf16_bf16_bf16_b4_g64")
    assert_out(got, O.aq_matmul(x, packed, s, b, N, K), EPS["bf16"], "bf16", "archive q4 matmul")
    td = pa.Tensor.empty([1, 64], "bf16")
    enc.encode(pa.Kernels.Matmul(upload(pa, x, "bf16"), down, td, True))
    stream.synchronize()
    assert_out(download(td, stream).reshape(1, 64), O.matmul(x, dense, 1, K, 64, True).reshape(1, 64), EPS["bf16"],
               "bf16", "archive dense matmul")


# ---- decode forms with the layer glue -------------------------------------------

def _q4_products(x, w_pre, packed, s, b, N, K):
    """x W^T (W 4-bit) for each rounding outcome of the pre-norm (or x itself)."""
    import flips
    vs = flips.norm_candidates(x, w_pre, 1e-6, O.BF16) if w_pre is not None else [x]
    return [O.aq_matmul(v[None], packed, s, b, N, K).ravel() for v in vs]


@pytest.mark.parametrize("ot", ["bf16", "f32"])
@pytest.mark.parametrize("residual,prenorm", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("K,N", [(2304, 4096), (2048, 2304), (384, 77)])
def test_q4_decode_matvec_glue(env, ot, residual, prenorm, K, N):
    import flips
    pa, lib, stream, enc = env
    eps = 1e-6
    rng = np.random.default_rng(K + N)
    x_in = rounded(rng.standard_normal(K).astype(np.float32), "bf16")
    delta = rounded(3 * rng.standard_normal(K).astype(np.float32), "bf16")
    w_post = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    w_pre = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    packed, s, b, q = quantize_q4(0.02 * rng.standard_normal((N, K)).astype(np.float32))
    out = pa.Tensor.empty([N], ot)
    x_out = pa.Tensor.empty([K], "bf16")
    kw = {}
    if residual:
        kw.update(delta=upload(pa, delta, "bf16"), w_post=pa.Tensor.from_numpy(w_post), x_out=x_out)
    if prenorm:
        kw.update(w_pre=pa.Tensor.from_numpy(w_pre))
    k = pa.Kernels.DecodeMatvec(upload(pa, x_in, "bf16"), _qtensor(pa, packed, s, b, N, K), out, eps=eps, **kw)
    f = int(residual) + 2 * int(prenorm)
    assert k.function_names[0].startswith(f"q4_decode_matvec_bf16_{ot}_l") and k.function_names[0].endswith(f"_f{f}")
    enc.encode(k)
    stream.synchronize()
    x = x_in
    if residual:
        x = download(x_out, stream)
        flips.assert_any(x, flips.residual_candidates(x_in, delta, w_post, eps, O.BF16), EPS["bf16"], "bf16",
                         "q4 residual stream")
    flips.assert_any(download(out, stream), _q4_products(x, w_pre if prenorm else None, packed, s, b, N, K),
                     EPS["bf16"], ot, f"q4 decode matvec r{residual} p{prenorm} {K}x{N}")


def test_q4_decode_matvec_kv_scatter(env):
    import flips
    pa, lib, stream, enc = env
    eps, Nq, Nkv, Hd, S, pos, H = 1e-6, 8, 4, 256, 4352, 4096, 2304
    QW, KW = Nq * Hd, Nkv * Hd
    N = QW + 2 * KW
    rng = np.random.default_rng(12)
    x_in = rounded(rng.standard_normal(H).astype(np.float32), "bf16")
    delta = rounded(rng.standard_normal(H).astype(np.float32), "bf16")
    w_post = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    w_pre = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    packed, s, b, q = quantize_q4(0.02 * rng.standard_normal((N, H)).astype(np.float32))
    kc0 = rounded(rng.standard_normal((Nkv, S, Hd)).astype(np.float32), "bf16")
    vc0 = rounded(rng.standard_normal((Nkv, S, Hd)).astype(np.float32), "bf16")
    kc, vc = upload(pa, kc0, "bf16"), upload(pa, vc0, "bf16")
    tq, x_out = pa.Tensor.empty([QW], "bf16"), pa.Tensor.empty([H], "bf16")
    k = pa.Kernels.DecodeMatvec(upload(pa, x_in, "bf16"), _qtensor(pa, packed, s, b, N, H), tq,
                                delta=upload(pa, delta, "bf16"), w_post=pa.Tensor.from_numpy(w_post), x_out=x_out,
                                w_pre=pa.Tensor.from_numpy(w_pre), k_cache=kc, v_cache=vc,
                                position=pa.Tensor.from_numpy(np.array([pos], np.int32)), q_rows=QW, eps=eps)
    enc.encode(k)
    stream.synchronize()
    x = download(x_out, stream)
    kg, vg = download(kc, stream).reshape(Nkv, S, Hd), download(vc, stream).reshape(Nkv, S, Hd)
    got = np.concatenate([download(tq, stream).ravel(), kg[:, pos].ravel(), vg[:, pos].ravel()])
    flips.assert_any(got, _q4_products(x, w_pre, packed, s, b, N, H), EPS["bf16"], "bf16", "q4 qkv + scatter")
    others = np.ones(S, bool)
    others[pos] = False
    np.testing.assert_array_equal(kg[:, others], kc0[:, others])
    np.testing.assert_array_equal(vg[:, others], vc0[:, others])


def _q4_hidden(n, gq, uq, F, H):
    """flips.HiddenOutcomes for 4-bit gate and up weights on the normed n."""
    n = np.asarray(n, np.float32).ravel()
    n2 = n.astype(np.float64) ** 2
    sums, norms = [], []
    for packed, s, b, q in (gq, uq):
        sums.append(O.aq_matmul(n[None], packed, s, b, F, H).ravel().astype(np.float64))
        norms.append(np.sqrt(dequantize_q4(q, s, b).astype(np.float64) ** 2 @ n2))
    return flips.HiddenOutcomes(sums[0], sums[1], norms[0], norms[1], H, O.BF16)


@pytest.mark.parametrize("residual", [False, True])
@pytest.mark.parametrize("H,F", [(2304, 9216), (256, 512)])
def test_q4_gated_mlp(env, residual, H, F):
    import flips
    pa, lib, stream, enc = env
    eps = 1e-6
    rng = np.random.default_rng(H + F + int(residual))
    x_in = rounded(rng.standard_normal(H).astype(np.float32), "bf16")
    delta = rounded(rng.standard_normal(H).astype(np.float32), "bf16")
    w_post = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    gq = quantize_q4(0.02 * rng.standard_normal((F, H)).astype(np.float32))
    uq = quantize_q4(0.02 * rng.standard_normal((F, H)).astype(np.float32))
    dq = quantize_q4(0.02 * rng.standard_normal((H, F)).astype(np.float32))
    out, x_out, hid = pa.Tensor.empty([H], "bf16"), pa.Tensor.empty([H], "bf16"), pa.Tensor.empty([F], "bf16")
    qt = [_qtensor(pa, p_, s_, b_, n_, k_) for (p_, s_, b_, _), n_, k_ in ((gq, F, H), (uq, F, H), (dq, H, F))]
    res = dict(delta=upload(pa, delta, "bf16"), w_post=pa.Tensor.from_numpy(w_post), x_out=x_out) if residual \
        else dict(delta=None, w_post=None, x_out=None)
    k = pa.Kernels.GatedMLPResidual(upload(pa, x_in, "bf16"), res["delta"], res["w_post"], res["x_out"],
                                    pa.Tensor.from_numpy(nw), qt[0], qt[1], qt[2], out, eps=eps, hidden=hid)
    names = k.function_names
    assert names[0].startswith("q4_gate_up_bf16_l") and names[0].endswith("_res") == residual
    assert names[1].startswith("aq_qmv_fast_bf16_bf16_bf16_b4_g64")
    enc.encode(k)
    stream.synchronize()
    x = x_in
    if residual:
        x = download(x_out, stream)
        flips.assert_any(x, flips.residual_candidates(x_in, delta, w_post, eps, O.BF16), EPS["bf16"], "bf16",
                         "q4 mlp residual")
    got_h, got = download(hid, stream), download(out, stream)
    errors = []
    for n in flips.norm_candidates(x, nw, eps, O.BF16):
        try:
            # the hidden vector exactly (flips.HiddenOutcomes), the down
            # projection of the kernel's own hidden vector to the 2e-3 bar
            _q4_hidden(n, gq, uq, F, H).check(got_h, "q4 hidden")
            assert_out(got, O.aq_matmul(got_h[None], dq[0], dq[1], dq[2], H, F).ravel(), EPS["bf16"], "bf16",
                       "q4 down")
            return
        except AssertionError as e:
            errors.append(str(e))
    raise AssertionError(" | ".join(errors))
