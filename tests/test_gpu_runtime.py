"""GPU tests of the runtime surface: library lookup and caching, raw launch
with several constants blocks, encoder ordering and scratch, glue kernels."""
import struct

import numpy as np
import pytest

import oracle as O
from gpu_util import gpu_env

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def test_library_caches_functions(env):
    # Tests/PopcornTests/Internals/KernelLibraryTests.swift:5-13
    pa, lib, stream, enc = env
    a = lib.function("add")
    b = lib.function("add")
    assert a.handle == b.handle
    attrs = a.attributes()
    assert attrs["wave_size"] == 64 and attrs["max_threads_per_block"] >= 256


def test_library_unknown_function(env):
    # KernelLibraryTests.swift:15-21
    pa, lib, stream, enc = env
    with pytest.raises(pa.PopcornError) as e:
        lib.function("does_not_exist")
    assert e.value.code == pa.PopcornError.KERNEL_FUNCTION_NOT_FOUND
    with pytest.raises(pa.PopcornError) as e:
        enc.encode(pa.Kernels.Custom("does_not_exist", [pa.Tensor.empty([4])], [1], [], (1, 1, 1), (64, 1, 1)))
    assert e.value.code == pa.PopcornError.KERNEL_FUNCTION_NOT_FOUND


def test_device_info(env):
    pa = env[0]
    info = pa.device_info(0)
    assert info["arch"].startswith("gfx950")
    assert info["wave_size"] == 64
    assert info["compute_units"] >= 1


def test_raw_launch_and_custom_kernel(env):
    # a caller-built DispatchKernel (MultipleConstantsTest.swift:15-85 binds
    # tensors then constants): scalar_mul with ScalarMulConstants{count, scalar}
    pa, lib, stream, enc = env
    x = pa.Tensor.from_numpy(np.arange(10, dtype=np.float32))
    y = pa.Tensor.empty([10])
    consts = struct.pack("<If", 10, -2.0)
    lib.launch("scalar_mul", (1, 1, 1), (256, 1, 1), [x.ptr, y.ptr], [consts], stream=stream)
    stream.synchronize()
    assert y.numpy(stream).tolist() == [-2.0 * i for i in range(10)]
    z = pa.Tensor.empty([10])
    enc.encode(pa.Kernels.Custom("scalar_mul", [x, z], [1, 2], [struct.pack("<If", 10, 3.0)], (1, 1, 1), (256, 1, 1)))
    stream.synchronize()
    assert z.numpy(stream).tolist() == [3.0 * i for i in range(10)]


def test_encoder_orders_dependent_dispatches_and_reuses_scratch(env):
    # a chain of dependent kernels on one stream (RAW hazards the reference
    # would barrier on), and composite kernels borrowing and returning scratch
    pa, lib, stream, enc = env
    pool = pa.ScratchPool()
    e2 = pa.KernelCommandEncoder(lib, stream, scratch=pool)
    a = pa.Tensor.from_numpy(np.ones(1000, np.float32))
    b = pa.Tensor.empty([1000])
    k1 = pa.Kernels.ScalarMul(a, 2.0, b)
    k2 = pa.Kernels.Add(b, b, a)
    e2.encode([k1, k2, k1, k2])  # a = ((1*2)+(1*2)) ... twice
    stream.synchronize()
    np.testing.assert_array_equal(a.numpy(stream), np.full(1000, 16.0, np.float32))
    st = e2.stats()
    assert st["dispatches"] == 4 and st["hazards"] >= 3
    x = pa.Tensor.from_numpy(np.random.default_rng(0).standard_normal(50000).astype(np.float32))
    idx = pa.Tensor.empty([1], "i32")
    for _ in range(3):
        e2.encode(pa.Kernels.Argmax(x, idx))
    stream.synchronize()
    assert e2.stats()["scratch_borrows"] == 6
    first = pool.nbytes
    e2.encode(pa.Kernels.Argmax(x, idx))
    stream.synchronize()
    assert pool.nbytes == first  # reused, not regrown
    e2.close()


def test_embedding_gather_kat(env):
    # KernelsTests.swift:121-138
    pa, lib, stream, enc = env
    table = pa.Tensor.from_numpy(np.array([0, 0, 0, 0, 1, 2, 3, 4, -1, -2, -3, -4], np.float32).reshape(3, 4))
    ids = pa.Tensor.from_numpy(np.array([2, 0, 1], np.int32))
    out = pa.Tensor.empty([3, 4])
    enc.encode(pa.Kernels.EmbeddingGather(ids, table, out))
    stream.synchronize()
    assert out.numpy(stream).ravel().tolist() == [-1, -2, -3, -4, 0, 0, 0, 0, 1, 2, 3, 4]


def test_embedding_gather_bf16_rows(env):
    pa, lib, stream, enc = env
    V, H = 1000, 2304
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 65536, (V, H), dtype=np.uint32).astype(np.uint16)
    ids_h = np.array([999, 0, 17, 17, 5000], np.int32)  # 5000 is out of range -> zeros
    out = pa.Tensor.empty([5, H], "bf16")
    enc.encode(pa.Kernels.EmbeddingGather(pa.Tensor.from_numpy(ids_h), pa.Tensor.from_numpy(bits, "bf16"), out))
    stream.synchronize()
    got = out.numpy(stream)
    np.testing.assert_array_equal(got[:4], bits[ids_h[:4]])
    assert not got[4].any()


@pytest.mark.parametrize("N", [1, 5, 31, 4096, 256000, 300001, 2000003])
def test_argmax_vs_oracle(env, N):
    pa, lib, stream, enc = env
    x = O.normal(N, (3, N))
    if N > 5:
        x[1, N // 2] = x[1, N // 3] = x[1].max() + 1.0  # tie: the first index wins (Argmax.metal:7-9)
    if N > 4101:
        # a tie between two loads of one thread (4096 apart: consecutive
        # batches of its 16 loads when a slice is over 4096 long)
        x[2, 5] = x[2, 4101] = x[2].max() + 1.0
    idx = pa.Tensor.empty([3], "i32")
    enc.encode(pa.Kernels.Argmax(pa.Tensor.from_numpy(x), idx))
    stream.synchronize()
    np.testing.assert_array_equal(idx.numpy(stream), O.argmax(x))


def test_argmax_nan_first_element_keeps_zero(env):
    pa, lib, stream, enc = env
    x = np.array([[np.nan, 1.0, 5.0, 2.0], [0.0, np.nan, 3.0, 3.0]], np.float32)
    idx = pa.Tensor.empty([2], "i32")
    enc.encode(pa.Kernels.Argmax(pa.Tensor.from_numpy(x), idx))
    stream.synchronize()
    np.testing.assert_array_equal(idx.numpy(stream), O.argmax(x))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_fill_normal_moments(env, dtype):
    pa, lib, stream, enc = env
    t = pa.Tensor.empty([1 << 20], dtype)
    lib.fill_normal(t, seed=9, mean=1.0, std=0.5, stream=stream)
    stream.synchronize()
    raw = t.numpy(stream)
    x = raw if dtype == "f32" else O.from_bits(raw.view(np.uint16), {"bf16": O.BF16, "f16": O.F16}[dtype])
    assert abs(float(x.mean()) - 1.0) < 0.005
    assert abs(float(x.std()) - 0.5) < 0.005
    assert abs(float(np.mean(np.abs(x - 1.0) > 1.0)) - 0.0455) < 0.003
