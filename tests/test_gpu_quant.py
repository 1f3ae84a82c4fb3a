"""GPU parity of the block-affine 4-bit path (AffineQuantizedMatmul.metal,
AffineQuantizedEmbeddingGather.metal) against the oracle, through the C ABI:
the decode matvec (aq_qmv_fast), M > 1 rows, the any-shape kernel, and the
dequantizing gather."""
import numpy as np
import pytest

import oracle as O
from conftest import assert_out
from gpu_util import EPS, download, gpu_env, rounded, upload
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
    assert k.function_names == [f"aq_embedding_gather_bf16_{ot}_b4_g64"]
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
