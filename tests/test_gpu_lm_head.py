"""GPU parity of the long-output matvecs (N >= 32768, four rows per streamed
unit) against the oracle, at the LM-head shape of BASELINE config 4:
the tied head [256000, 2304] of Gemma4TextInference.swift:201-206, which the
reference runs as Kernels.Matmul with m == 1 -> matvec_nk_simd4
(Matmul.swift:240-251, Matvec.metal:55-137).

Covered: the plain Matmul route (bf16 -> bf16 and bf16 -> f32) at N = 32768,
32771 (a ragged last unit) and 256000; the decode matvec with the residual
add and the final norm in front (the decoder's head kernel); and the 4-bit
head (block-affine weights, group 64). Large weights are filled on the
device (popcorn_fill_normal) and read back, so the oracle and the GPU see
the same bytes; integer-valued weights give results that are exact in f32
whatever the summation order, which pins every row's index bit for bit."""
import numpy as np
import pytest

import oracle as O
import flips
from conftest import assert_out
from flips import assert_any
from gpu_util import EPS, download, gpu_env, rounded, upload

pytestmark = pytest.mark.gpu

K = 2304
BF16_OF_INT = (np.arange(-8, 9, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)  # exact bf16 of -8..8


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def _device_normal(env, shape, seed, std):
    """A bf16 tensor of N(0, std) filled on the device, and its f32 values."""
    pa, lib, stream, enc = env
    t = pa.Tensor.empty(list(shape), "bf16")
    lib.fill_normal(t, seed, 0.0, std, stream)
    stream.synchronize()
    bits = t.numpy(stream).view(np.uint16)
    return t, (bits.astype(np.uint32) << 16).view(np.float32)


def _int_weights(N, seed):
    rng = np.random.default_rng(seed)
    w = rng.integers(-8, 9, size=(N, K), dtype=np.int8)
    return w, BF16_OF_INT[w + 8]


def _exact_product(w_int8, x):
    """x . W^T for integer-valued inputs with every partial sum below 2^24: exact in f32."""
    y = np.empty(w_int8.shape[0], np.float32)
    for i in range(0, w_int8.shape[0], 32768):
        y[i:i + 32768] = w_int8[i:i + 32768].astype(np.float32) @ x
    return y


@pytest.mark.parametrize("N", [32768, 32771, 256000])
def test_matmul_r4_integer_exact(env, N):
    pa, lib, stream, enc = env
    w_int, w_bits = _int_weights(N, N)
    x = np.random.default_rng(N + 1).integers(-4, 5, size=K).astype(np.float32)  # |sum| <= 73728
    tw = pa.Tensor.from_numpy(w_bits, "bf16")
    tx = upload(pa, x[None, :], "bf16")
    want = _exact_product(w_int, x)
    for ot in ("f32", "bf16"):
        out = pa.Tensor.empty([1, N], ot)
        k = pa.Kernels.Matmul(tx, tw, out, True)
        assert k.function_names == [f"matvec_nk_stream_bf16_bf16_{ot}_r4"]
        enc.encode(k)
        stream.synchronize()
        got = download(out, stream).ravel()
        # the sum is exact, so the stored result is the exact value rounded once
        np.testing.assert_array_equal(got, rounded(want, ot), err_msg=f"N={N} out={ot}")


@pytest.mark.parametrize("N", [32771, 256000])
def test_matmul_r4_vs_oracle(env, N):
    pa, lib, stream, enc = env
    tw, w = _device_normal(env, (N, K), seed=N, std=0.02)
    x = rounded(O.normal(N + 7, (1, K)), "bf16")
    tx = upload(pa, x, "bf16")
    ref = O.matmul(x, w, 1, K, N, True)
    for ot in ("bf16", "f32"):
        out = pa.Tensor.empty([1, N], ot)
        enc.encode(pa.Kernels.Matmul(tx, tw, out, True))
        stream.synchronize()
        assert_out(download(out, stream), ref, EPS["bf16"], ot, f"LM-head matvec N={N} bf16->{ot}")


def test_decode_matvec_lm_head_residual_final_norm(env):
    # the decoder's head: x = x_in + RMSNorm(delta) * w_post (the last layer's
    # post-FFN norm and residual Add), then logits = RMSNorm(x; final norm) . E^T
    # in f32 (Gemma4TextInference.swift:430-434, :195-206)
    pa, lib, stream, enc = env
    N, eps = 256000, 1e-6
    tw, w = _device_normal(env, (N, K), seed=11, std=0.02)
    x_in = rounded(O.normal(12, (K,)), "bf16")
    delta = rounded(O.normal(13, (K,), std=3.0), "bf16")
    w_post = O.normal(14, (K,), mean=1.0, std=0.1)
    w_pre = O.normal(15, (K,), mean=1.0, std=0.1)
    out = pa.Tensor.empty([N], "f32")
    x_out = pa.Tensor.empty([K], "bf16")
    k = pa.Kernels.DecodeMatvec(upload(pa, x_in, "bf16"), tw, out, delta=upload(pa, delta, "bf16"),
                                w_post=pa.Tensor.from_numpy(w_post), x_out=x_out, w_pre=pa.Tensor.from_numpy(w_pre),
                                eps=eps)
    assert k.function_names == ["decode_matvec_bf16_f32_r4_f3"]
    enc.encode(k)
    stream.synchronize()
    x = download(x_out, stream)
    assert_any(x, flips.residual_candidates(x_in, delta, w_post, eps, O.BF16), EPS["bf16"], "bf16",
               "head residual stream")
    refs = [O.matmul(v, w, 1, K, N, True).ravel() for v in flips.norm_candidates(x, w_pre, eps, O.BF16)]
    assert_any(download(out, stream), refs, EPS["bf16"], "f32", "LM head logits (residual + final norm)")


def test_quantized_lm_head(env):
    # 4-bit tied head (MLX block-affine, group 64, bf16 scales and biases):
    # the Matmul route (m == 1) and the decoder's glued form with the final
    # norm in front, both against the oracle's dequantized product
    pa, lib, stream, enc = env
    N, eps = 256000, 1e-6
    rng = np.random.default_rng(21)
    packed = rng.integers(0, 2 ** 32, (N, K // 8), dtype=np.uint32)
    s = O.round_to(rng.uniform(0.002, 0.004, (N, K // 64)).astype(np.float32), O.BF16)
    b = O.round_to(rng.uniform(-0.04, -0.02, (N, K // 64)).astype(np.float32), O.BF16)
    qt = pa.AffineQuantizedTensor(pa.Tensor.from_numpy(packed, "u32"), upload(pa, s, "bf16"), upload(pa, b, "bf16"),
                                  [N, K])
    x = rounded(O.normal(22, (1, K)), "bf16")
    ref = O.aq_matmul(x, packed, s, b, N, K)
    out = pa.Tensor.empty([1, N], "f32")
    k = pa.Kernels.Matmul(upload(pa, x, "bf16"), qt, out)
    assert k.function_names[0].startswith("aq_qmv_fast_bf16_bf16_f32_b4_g64_l")
    enc.encode(k)
    stream.synchronize()
    assert_out(download(out, stream), ref, EPS["bf16"], "f32", "4-bit LM head (Matmul)")

    w_pre = O.normal(23, (K,), mean=1.0, std=0.1)
    logits = pa.Tensor.empty([N], "f32")
    k = pa.Kernels.DecodeMatvec(upload(pa, x.ravel(), "bf16"), qt, logits, w_pre=pa.Tensor.from_numpy(w_pre), eps=eps)
    assert k.function_names[0].startswith("q4_decode_matvec_bf16_f32_l") and k.function_names[0].endswith("_f2")
    enc.encode(k)
    stream.synchronize()
    refs = [O.aq_matmul(v[None, :], packed, s, b, N, K).ravel()
            for v in flips.norm_candidates(x.ravel(), w_pre, eps, O.BF16)]
    assert_any(download(logits, stream), refs, EPS["bf16"], "f32", "4-bit LM head (final norm glued)")
