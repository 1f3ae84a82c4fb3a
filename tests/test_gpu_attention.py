"""GPU parity: FlashAttention router -> split-KV decoding (FlashDecoding +
combine) and the plain prefill path, through the C ABI, against the oracle's
naive attention (the generalised reference test loop)."""
import numpy as np
import pytest

import oracle as O
from conftest import assert_approx, assert_out
from gpu_util import EPS, download, gpu_env, rounded, upload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def _attend(env, q, k, v, dtype, out_dtype, scale, mask=None, key_len=None, position=None):
    pa, lib, stream, enc = env
    B, Nq, Sq, Hd = q.shape
    Nkv, cap = k.shape[1], k.shape[2]
    Sk = cap if key_len is None else key_len
    mask = mask or pa.AttentionMask.causal
    tq, tk, tv = upload(pa, q, dtype), upload(pa, k, dtype), upload(pa, v, dtype)
    to = pa.Tensor.empty([B, Nq, Sq, Hd], out_dtype)
    pos_t = pa.Tensor.from_numpy(np.array([position], np.int32)) if position is not None else None
    kern = pa.Kernels.FlashAttention(tq, tk, tv, out=to, scale=scale, mask=mask, batch=B, query_heads=Nq,
                                     kv_heads=Nkv, query_len=Sq, key_len=Sk, head_dim=Hd, key_capacity=cap,
                                     position=pos_t)
    enc.encode(kern)
    stream.synchronize()
    return download(to, stream), kern


def _inputs(seed, B, Nq, Nkv, Sq, cap, Hd, dtype, std=1.0):
    q = rounded(O.normal(seed, (B, Nq, Sq, Hd), std=std), dtype)
    k = rounded(O.normal(seed + 1, (B, Nkv, cap, Hd), std=std), dtype)
    v = rounded(O.normal(seed + 2, (B, Nkv, cap, Hd)), dtype)
    return q, k, v


def test_config1_tiny_f32_decode(env):
    # BASELINE config 1 attention: Nq 4, Nkv 1, Hd 64, 129 keys (128 + the new one), scale 1/8
    q, k, v = _inputs(100, 1, 4, 1, 1, 129, 64, "f32")
    got, kern = _attend(env, q, k, v, "f32", "f32", 0.125)
    assert kern.function_names[0] == "flash_decoding_partial_f32_l16_c1_g4"
    assert_approx(got, O.attention_naive(q, k, v, 0.125), EPS["f32"], "config 1 attention")


def test_gemma_decode_bf16_with_capacity(env):
    # config 4 shape: 8 q heads, 4 KV heads (GQA 2:1), Hd 256, cache capacity 4352, 4097 keys used
    q, k, v = _inputs(200, 1, 8, 4, 1, 4352, 256, "bf16")
    got, kern = _attend(env, q, k, v, "bf16", "bf16", 1 / 16, key_len=4097)
    assert kern.function_names == ["flash_decoding_partial_bf16_l32_c1_g2_w8", "flash_decoding_reduce_bf16_ext"]
    assert_out(got, O.attention_naive(q, k, v, 1 / 16, key_len=4097), EPS["bf16"], "bf16", "gemma decode")


@pytest.mark.parametrize("B,ctx", [(1, 2048), (8, 2048), (1, 8192), (8, 8192), (32, 2048)])
def test_config2_f16_decode(env, B, ctx):
    # Q [B,8,1,256], KV [B,4,ctx,256] N(0,1), scale 1/16, no mask
    q, k, v = _inputs(300 + B + ctx, B, 8, 4, 1, ctx, 256, "f16")
    got, _ = _attend(env, q, k, v, "f16", "f16", 1 / 16, mask=env[0].AttentionMask.bidirectional)
    assert_out(got, O.attention_naive(q, k, v, 1 / 16, mask_kind=2), EPS["f16"], "f16", f"config 2 B={B} ctx={ctx}")


@pytest.mark.parametrize("B,ctx", [(1, 32768), (8, 32768), (32, 8192), (32, 32768)])
def test_config2_f16_large_sampled(env, B, ctx):
    # the config-2 points too large for host-generated inputs (up to 4.3 GB
    # of KV): inputs filled on the device, the GPU runs the whole batch, the
    # oracle checks the first, a middle and the last batch entry (attention is
    # independent per entry) on the same bytes.
    pa, lib, stream, enc = env
    Nq, Nkv, Hd = 8, 4, 256
    tq = pa.Tensor.empty([B, Nq, 1, Hd], "f16")
    tk = pa.Tensor.empty([B, Nkv, ctx, Hd], "f16")
    tv = pa.Tensor.empty([B, Nkv, ctx, Hd], "f16")
    for i, t in enumerate((tq, tk, tv)):
        lib.fill_normal(t, seed=400 + 7 * B + ctx + i, stream=stream)
    to = pa.Tensor.empty([B, Nq, 1, Hd], "f16")
    enc.encode(pa.Kernels.FlashAttention(tq, tk, tv, to, scale=1 / 16, mask=pa.AttentionMask.bidirectional))
    stream.synchronize()
    got = download(to, stream)
    per_b = Nkv * ctx * Hd
    for b in sorted({0, B // 2, B - 1}):
        q = download(tq.view([1, Nq, 1, Hd], offset_elements=b * Nq * Hd), stream)
        k = download(tk.view([1, Nkv, ctx, Hd], offset_elements=b * per_b), stream)
        v = download(tv.view([1, Nkv, ctx, Hd], offset_elements=b * per_b), stream)
        assert abs(float(k.std()) - 1.0) < 0.01
        ref = O.attention_naive(q, k, v, 1 / 16, mask_kind=2)
        assert_out(got[b:b + 1], ref, EPS["f16"], "f16", f"config 2 B={B} ctx={ctx} b={b}")


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("Nq,Nkv,Hd", [(8, 8, 64), (8, 4, 128), (6, 2, 256), (16, 2, 128), (16, 1, 64),
                                        (4, 2, 512), (2, 1, 80), (3, 3, 32)])
def test_decode_head_layouts(env, dtype, Nq, Nkv, Hd):
    cap, Sk = 700, 611
    q, k, v = _inputs(Nq * 10 + Hd, 2, Nq, Nkv, 1, cap, Hd, dtype)
    got, _ = _attend(env, q, k, v, dtype, dtype, 1 / np.sqrt(Hd), key_len=Sk)
    assert_out(got, O.attention_naive(q, k, v, 1 / np.sqrt(Hd), key_len=Sk), EPS[dtype], dtype, f"{dtype} {Nq}/{Nkv}/{Hd}")


@pytest.mark.parametrize("Sk", [1, 2, 63, 64, 65, 129, 1000])
def test_decode_short_and_ragged_contexts(env, Sk):
    q, k, v = _inputs(500 + Sk, 1, 8, 4, 1, Sk, 256, "bf16")
    got, _ = _attend(env, q, k, v, "bf16", "f32", 1 / 16)
    assert_approx(got, O.attention_naive(q, k, v, 1 / 16), 2e-3, f"Sk={Sk}")


def test_decode_sliding_window(env):
    pa = env[0]
    q, k, v = _inputs(600, 1, 8, 4, 1, 3000, 256, "bf16")
    got, _ = _attend(env, q, k, v, "bf16", "bf16", 1 / 16, mask=pa.AttentionMask.causal_sliding_window(512))
    ref = O.attention_naive(q, k, v, 1 / 16, mask_kind=1, window=512)
    assert_out(got, ref, 2e-3, "bf16", "sliding window")


def test_decode_position_tensor_matches_static(env):
    # position p => key_len = p + 1 read on the device (graph replay path)
    q, k, v = _inputs(700, 1, 8, 4, 1, 4352, 256, "bf16")
    for p in (0, 1000, 4096, 4351):
        got, _ = _attend(env, q, k, v, "bf16", "bf16", 1 / 16, key_len=1, position=p)
        ref = O.attention_naive(q, k, v, 1 / 16, key_len=p + 1)
        assert_out(got, ref, 2e-3, "bf16", f"position {p}")


def test_reference_bidirectional_fa_case(env):
    # BidirectionalFATests.swift:90-150: b1 h2 sq96 hd64 f32, xorshift inputs,
    # maxAbs < 1e-3 against the naive reference, causal NaN-free
    pa = env[0]
    total = 2 * 96 * 64
    qkv = O.fa_test_floats(0xDEADBEEFCAFEBABE, 3 * total)
    q, k, v = (qkv[i * total:(i + 1) * total].reshape(1, 2, 96, 64) for i in range(3))
    got, kern = _attend(env, q, k, v, "f32", "f32", 1 / 8, mask=pa.AttentionMask.bidirectional)
    assert pa.Kernels.route(96, 64, "f32") in ("plain", "tiled")
    expected = O.attention_naive(q, k, v, 1 / 8, mask_kind=2)
    assert not np.isnan(got).any()
    assert np.abs(got - expected).max() < 1e-3
    assert_approx(got, expected, 1e-5, "bidirectional f32")
    causal, _ = _attend(env, q, k, v, "f32", "f32", 1 / 8)
    assert not np.isnan(causal).any()
    assert_approx(causal, O.attention_naive(q, k, v, 1 / 8), 1e-5, "causal f32")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_prefill_causal_sq_ne_sk(env, dtype):
    # causal with Sq < Sk: posQ = Sk - Sq + i (FlashAttention.metal:72)
    q, k, v = _inputs(800, 1, 4, 2, 37, 300, 128, dtype)
    got, _ = _attend(env, q, k, v, dtype, dtype, 0.1)
    assert_out(got, O.attention_naive(q, k, v, 0.1), EPS[dtype], dtype, "prefill causal")


def test_attention_validation(env):
    pa = env[0]
    q = pa.Tensor.empty([1, 3, 1, 64])
    k = pa.Tensor.empty([1, 2, 10, 64])
    with pytest.raises(pa.PopcornError) as e:
        pa.Kernels.FlashAttention(q, k, k, pa.Tensor.empty([1, 3, 1, 64]), scale=1.0)
    assert e.value.code == pa.PopcornError.TENSOR_SHAPE_MISMATCH
    with pytest.raises(pa.PopcornError) as e:
        pa.Kernels.FlashAttention(pa.Tensor.empty([1, 2, 1, 64]), k, pa.Tensor.empty([1, 2, 11, 64]),
                                  pa.Tensor.empty([1, 2, 1, 64]), scale=1.0)
    assert e.value.code == pa.PopcornError.TENSOR_SHAPE_MISMATCH
    with pytest.raises(pa.PopcornError) as e:
        pa.Kernels.FlashAttention(pa.Tensor.empty([1, 2, 1, 64]), pa.Tensor.empty([1, 2, 10, 64], "bf16"),
                                  pa.Tensor.empty([1, 2, 10, 64], "bf16"), pa.Tensor.empty([1, 2, 1, 64]), scale=1.0)
    assert e.value.code == pa.PopcornError.UNSUPPORTED_DATA_TYPE_COMBINATION
