"""BASELINE config 1 as one encoded sequence on the GPU, against the oracle.

The tiny f32 decoder-layer step: hidden 256, 4 query heads, 1 KV head, head
dim 64, SwiGLU FFN 1024, a KV cache holding 128 rows; weights N(0, 0.02),
activations and cache N(0, 1), RMSNorm weight 1 + N(0, 0.1), eps 1e-6, scale
1/sqrt(64), seed 0. One encoder sequence writes the new K and V rows at
position 128 (KVCacheWrite.swift:37-48), runs FlashDecoding over the 129 keys
(FlashDecoding.swift:54-73, through the FlashAttention router) and feeds the
[4 x 64] = [256] attention output to the gated MLP (RMSNorm, gate and up,
GELU-tanh(gate) * up, down; Gemma4TextInference.swift:416-429). The KV write
is held bit-exact; every other stage to the f32 bar (1e-5), both on the
GPU's own input to that stage and end to end against the oracle's whole
composition."""
import numpy as np
import pytest

import oracle as O
from conftest import assert_approx
from gpu_util import download, gpu_env, upload

pytestmark = pytest.mark.gpu

H, NQ, NKV, HD, F, CTX = 256, 4, 1, 64, 1024, 128


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def _inputs(seed=0):
    """Config 1's tensors from one seed (the oracle's generator, f32)."""
    g = iter(range(seed * 100, seed * 100 + 100))
    cache_k = np.zeros((1, NKV, CTX + 1, HD), np.float32)
    cache_v = np.zeros((1, NKV, CTX + 1, HD), np.float32)
    cache_k[:, :, :CTX] = O.normal(next(g), (1, NKV, CTX, HD))
    cache_v[:, :, :CTX] = O.normal(next(g), (1, NKV, CTX, HD))
    return dict(
        k_new=O.normal(next(g), (1, NKV, 1, HD)), v_new=O.normal(next(g), (1, NKV, 1, HD)),
        q=O.normal(next(g), (1, NQ, 1, HD)), cache_k=cache_k, cache_v=cache_v,
        norm_w=O.normal(next(g), (H,), mean=1.0, std=0.1),
        w_gate=O.normal(next(g), (F, H), std=0.02), w_up=O.normal(next(g), (F, H), std=0.02),
        w_down=O.normal(next(g), (H, F), std=0.02))


def test_config1_step_as_one_sequence(env):
    pa, lib, stream, enc = env
    x = _inputs(0)
    t = {n: upload(pa, a, "f32") for n, a in x.items()}
    attn = pa.Tensor.empty([1, NQ, 1, HD], "f32")
    mlp_in = attn.view([H])
    out = pa.Tensor.empty([H], "f32")
    hidden = pa.Tensor.empty([F], "f32")
    scale = 1.0 / np.sqrt(HD)
    kernels = [
        pa.Kernels.KVCacheWrite(t["k_new"], t["cache_k"], CTX),
        pa.Kernels.KVCacheWrite(t["v_new"], t["cache_v"], CTX),
        pa.Kernels.FlashAttention(t["q"], t["cache_k"], t["cache_v"], attn, scale=scale),
        pa.Kernels.GatedMLP(mlp_in, t["norm_w"], t["w_gate"], t["w_up"], t["w_down"], out, eps=1e-6, hidden=hidden),
    ]
    assert [k.function_names[0] for k in kernels] == [
        "kv_cache_write", "kv_cache_write", "flash_decoding_partial_f32_l16_c1_g4", "gated_mlp_gate_up_f32_r1"]
    enc.encode(kernels)  # the result-builder form: one ordered sequence
    stream.synchronize()

    # KV write: bit-exact (KVCacheWrite.metal; KernelsTests.swift:551-564's semantics)
    ck, cv = x["cache_k"].copy(), x["cache_v"].copy()
    assert O.kv_cache_write(x["k_new"], O.F32, ck, O.F32, CTX) == 0
    assert O.kv_cache_write(x["v_new"], O.F32, cv, O.F32, CTX) == 0
    np.testing.assert_array_equal(download(t["cache_k"], stream), ck)
    np.testing.assert_array_equal(download(t["cache_v"], stream), cv)

    # attention over the 129 keys, on the caches just checked
    a_ref = O.attention_naive(x["q"], ck, cv, scale)
    a_gpu = download(attn, stream)
    assert_approx(a_gpu, a_ref, 1e-5, "config 1 attention")
    # FlashDecoding equals naive attention for the reference's P = 8 too
    assert_approx(O.flash_decoding(x["q"], ck, cv, scale, 8), a_ref, 1e-5, "oracle FD P=8")

    # the MLP on the GPU's attention output, then end to end
    h_ref, y_ref = O.gated_mlp(a_gpu.reshape(H), x["norm_w"], 1e-6, x["w_gate"], x["w_up"], x["w_down"])
    assert_approx(download(hidden, stream), h_ref, 1e-5, "config 1 gated hidden")
    assert_approx(download(out, stream), y_ref, 1e-5, "config 1 MLP out")
    _, y_e2e = O.gated_mlp(a_ref.reshape(H), x["norm_w"], 1e-6, x["w_gate"], x["w_up"], x["w_down"])
    assert_approx(download(out, stream), y_e2e, 1e-5, "config 1 end to end")
