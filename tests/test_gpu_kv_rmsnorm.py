"""GPU parity: KV-cache write (bit-exact) and RMSNorm, through the C ABI."""
import zlib

import numpy as np
import pytest

import oracle as O
from conftest import assert_approx, assert_out
from gpu_util import EPS, TAG, download, gpu_env, rounded, upload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def test_kv_cache_write_reference_kat(env):
    # Tests/PopcornTests/Kernels/KernelsTests.swift:551-564
    pa, lib, stream, enc = env
    src = pa.Tensor.from_numpy(np.array([1, 2, 3, 4], np.float32).reshape(1, 1, 2, 2))
    cache = pa.Tensor.from_numpy(np.zeros((1, 1, 4, 2), np.float32))
    enc.encode(pa.Kernels.KVCacheWrite(src, cache, offset=1))
    stream.synchronize()
    assert cache.numpy(stream).ravel().tolist() == [0, 0, 1, 2, 3, 4, 0, 0]


@pytest.mark.parametrize("src_t,cache_t", [("f32", "f32"), ("bf16", "bf16"), ("f32", "bf16"), ("f16", "f16")])
@pytest.mark.parametrize("shape,smax,offset", [((1, 4, 1, 256), 4352, 4096), ((2, 3, 5, 64), 11, 6),
                                               ((1, 2, 3, 7), 9, 2), ((3, 1, 17, 12), 40, 23)])
def test_kv_cache_write_bit_exact(env, src_t, cache_t, shape, smax, offset):
    pa, lib, stream, enc = env
    B, Nkv, Snew, Hd = shape
    rng = np.random.default_rng(zlib.crc32(repr((src_t, cache_t, shape)).encode()))
    if src_t == "f32":
        src_host = rng.standard_normal(shape).astype(np.float32)
        # include rounding ties and the NaN -> Inf quirk of the bf16 store formula
        flat = src_host.reshape(-1)
        flat[:4] = np.array([0x3F808000, 0x3F818000, 0x7F800001, 0xFF7FFFFF], np.uint32).view(np.float32)
    else:
        src_host = rng.integers(0, 65536, shape, dtype=np.uint32).astype(np.uint16)  # any bits, NaNs included
    init = rng.integers(0, 65536, (B, Nkv, smax, Hd), dtype=np.uint32)
    cache_host = init.astype(np.float32) if cache_t == "f32" else init.astype(np.uint16)
    expect = cache_host.copy()
    assert O.kv_cache_write(src_host, TAG[src_t], expect, TAG[cache_t], offset) == 0
    src = pa.Tensor.from_numpy(src_host, src_t)
    cache = pa.Tensor.from_numpy(cache_host, cache_t)
    enc.encode(pa.Kernels.KVCacheWrite(src, cache, offset=offset))
    stream.synchronize()
    got = cache.numpy(stream)
    np.testing.assert_array_equal(got.view(np.uint32 if cache_t == "f32" else np.uint16),
                                  expect.view(np.uint32 if cache_t == "f32" else np.uint16))


def test_kv_cache_write_position_tensor(env):
    pa, lib, stream, enc = env
    B, Nkv, Hd, smax = 1, 4, 256, 64
    rng = np.random.default_rng(7)
    src_host = rng.integers(0, 65536, (B, Nkv, 1, Hd), dtype=np.uint32).astype(np.uint16)
    cache = pa.Tensor.from_numpy(np.zeros((B, Nkv, smax, Hd), np.uint16), "bf16")
    src = pa.Tensor.from_numpy(src_host, "bf16")
    pos = pa.Tensor.from_numpy(np.array([37], np.int32))
    k = pa.Kernels.KVCacheWrite(src, cache, position=pos)
    enc.encode(k)
    stream.synchronize()
    expect = np.zeros((B, Nkv, smax, Hd), np.uint16)
    expect[:, :, 37] = src_host[:, :, 0]
    np.testing.assert_array_equal(cache.numpy(stream), expect)
    # a position past the capacity writes nothing
    pos.copy_from(np.array([smax], np.int32))
    enc.encode(k)
    stream.synchronize()
    np.testing.assert_array_equal(cache.numpy(stream), expect)


def test_kv_cache_write_validation(env):
    pa, lib, stream, enc = env
    src = pa.Tensor.empty([1, 1, 2, 2])
    cache = pa.Tensor.empty([1, 1, 4, 2])
    with pytest.raises(pa.PopcornError) as e:
        pa.Kernels.KVCacheWrite(src, cache, offset=3)
    assert e.value.code == pa.PopcornError.TENSOR_SHAPE_MISMATCH
    with pytest.raises(pa.PopcornError) as e:
        pa.Kernels.KVCacheWrite(pa.Tensor.empty([1, 1, 2, 2], "bf16"), pa.Tensor.empty([1, 1, 4, 2], "f16"), offset=0)
    assert e.value.code == pa.PopcornError.UNSUPPORTED_DATA_TYPE_COMBINATION


# ---- RMSNorm ------------------------------------------------------------------

def test_rmsnorm_reference_kats(env):
    pa, lib, stream, enc = env
    # KernelsTests.swift:142-162
    x = pa.Tensor.from_numpy(np.array([1, 2, 3, 4], np.float32))
    w = pa.Tensor.from_numpy(np.zeros(4, np.float32))
    out = pa.Tensor.empty([4])
    enc.encode(pa.Kernels.RMSNorm(x, w, out, row_count=1, hidden_size=4, eps=1e-6, add_one_to_weight=True))
    # KernelsTests.swift:164-175
    x2 = pa.Tensor.from_numpy(np.array([[3, 4]], np.float32))
    out2 = pa.Tensor.empty([1, 2])
    enc.encode(pa.Kernels.RMSNorm(x2, None, out2, eps=0.0))
    stream.synchronize()
    assert_approx(out.numpy(stream), np.array([1, 2, 3, 4]) / np.sqrt(7.5), 1e-4, "gemma kat")
    assert_approx(out2.numpy(stream).ravel(), np.array([3, 4]) / np.sqrt(12.5), 1e-4, "no-weight kat")


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,H,weight,add_one", [(1, 2304, True, False), (1, 256, True, True), (7, 2304, True, False),
                                                   (300, 640, False, False), (2, 777, True, False), (1, 3072, True, True)])
def test_rmsnorm_vs_oracle(env, dtype, rows, H, weight, add_one):
    pa, lib, stream, enc = env
    x = rounded(O.normal(rows * 31 + H, (rows, H)), dtype)
    w = O.normal(H, (H,), mean=0.0 if add_one else 1.0, std=0.1) if weight else None
    tx = upload(pa, x, dtype)
    tw = pa.Tensor.from_numpy(w) if weight else None
    out = pa.Tensor.empty([rows, H], dtype)
    enc.encode(pa.Kernels.RMSNorm(tx, tw, out, eps=1e-6, add_one_to_weight=add_one))
    stream.synchronize()
    ref = O.rmsnorm(x, w, 1e-6, add_one)
    assert_out(download(out, stream), ref, EPS[dtype], dtype, f"rmsnorm {dtype} {rows}x{H}")


def test_rmsnorm_validation(env):
    pa, lib, stream, enc = env
    x = pa.Tensor.empty([2, 8])
    with pytest.raises(pa.PopcornError) as e:
        pa.Kernels.RMSNorm(x, None, pa.Tensor.empty([2, 8]), axis=0, eps=1e-6)
    assert e.value.code == pa.PopcornError.TENSOR_INVALID_AXIS
    with pytest.raises(pa.PopcornError) as e:
        pa.Kernels.RMSNorm(x, pa.Tensor.empty([7]), pa.Tensor.empty([2, 8]), eps=1e-6)
    assert e.value.code == pa.PopcornError.TENSOR_SHAPE_MISMATCH
