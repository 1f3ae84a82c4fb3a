"""GPU test of the allocation-free split-KV attention
(popcorn_flash_decoding_no_alloc, include/popcorn_hip.h), called through
the C ABI: its output equals the descriptor path's (popcorn_kernel_flash_
attention_dims + encode, the same kernels on a borrowed scratch buffer) bit
for bit, on two calls in a row with the second smaller, and a shape whose
partials exceed the static scratch is refused with workspaceExhausted
before anything runs."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from gpu_util import download, gpu_env, rounded, upload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def _no_alloc(pa, lib, stream, q, k, v, out, B, Nq, Nkv, Sq, Sk, Hd, scale, cap, position=None):
    from popcorn_amd import runtime as R

    mask = pa.AttentionMask.causal.desc()
    pos = C.byref(position.desc()) if position is not None else None
    R.check(R.lib().popcorn_flash_decoding_no_alloc(lib.handle, R._stream_handle(stream), C.byref(q.desc()),
                                                    C.byref(k.desc()), C.byref(v.desc()), C.byref(out.desc()), B, Nq,
                                                    Nkv, Sq, Sk, Hd, scale, mask, cap, pos))


CASES = [  # (dtype, B, Nq, Nkv, Sq, Sk, cap, Hd): the decode step's shape first, then a smaller one
    ("bf16", 2, 8, 4, 1, 4097, 4352, 256),
    ("f32", 1, 4, 1, 1, 129, 129, 64),
]


def test_no_alloc_attention_equals_descriptor_path(env):
    pa, lib, stream, enc = env
    for i, (t, B, Nq, Nkv, Sq, Sk, cap, Hd) in enumerate(CASES):
        scale = 1.0 / np.sqrt(Hd)
        q = rounded(O.normal(10 + i, (B, Nq, Sq, Hd)), t)
        k = rounded(O.normal(20 + i, (B, Nkv, cap, Hd)), t)
        v = rounded(O.normal(30 + i, (B, Nkv, cap, Hd)), t)
        tq, tk, tv = upload(pa, q, t), upload(pa, k, t), upload(pa, v, t)
        want = pa.Tensor.empty([B, Nq, Sq, Hd], t)
        enc.encode(pa.Kernels.FlashAttention(tq, tk, tv, out=want, scale=scale, batch=B, query_heads=Nq,
                                             kv_heads=Nkv, query_len=Sq, key_len=Sk, head_dim=Hd, key_capacity=cap))
        got = pa.Tensor.empty([B, Nq, Sq, Hd], t)
        _no_alloc(pa, lib, stream, tq, tk, tv, got, B, Nq, Nkv, Sq, Sk, Hd, scale, cap)
        stream.synchronize()
        np.testing.assert_array_equal(got.numpy(stream), want.numpy(stream), err_msg=f"case {i}")
        # and both are the oracle's attention
        ref = O.attention_naive(q, k, v, scale, key_len=Sk)
        assert np.abs(download(got, stream) - ref).max() < (2e-2 if t == "bf16" else 1e-5)


def test_no_alloc_attention_with_device_position(env):
    # the graph-replay form: key length from a position tensor
    pa, lib, stream, enc = env
    B, Nq, Nkv, Hd, cap = 1, 8, 4, 256, 4352
    q = rounded(O.normal(41, (B, Nq, 1, Hd)), "bf16")
    k = rounded(O.normal(42, (B, Nkv, cap, Hd)), "bf16")
    v = rounded(O.normal(43, (B, Nkv, cap, Hd)), "bf16")
    tq, tk, tv = upload(pa, q, "bf16"), upload(pa, k, "bf16"), upload(pa, v, "bf16")
    for p in (4096, 100):
        pos = pa.Tensor.from_numpy(np.array([p], np.int32))
        want = pa.Tensor.empty([B, Nq, 1, Hd], "bf16")
        enc.encode(pa.Kernels.FlashAttention(tq, tk, tv, out=want, scale=1 / 16, batch=B, query_heads=Nq,
                                             kv_heads=Nkv, query_len=1, key_len=1, head_dim=Hd, key_capacity=cap,
                                             position=pos))
        got = pa.Tensor.empty([B, Nq, 1, Hd], "bf16")
        _no_alloc(pa, lib, stream, tq, tk, tv, got, B, Nq, Nkv, 1, 1, Hd, 1 / 16, cap, position=pos)
        stream.synchronize()
        np.testing.assert_array_equal(got.numpy(stream), want.numpy(stream), err_msg=f"position {p}")


def test_no_alloc_attention_refuses_partials_beyond_the_scratch(env):
    # 64 batch entries x 8 heads x 64 rows x P partitions x (512 + 2) floats
    # is far above 4 MiB: refused before any launch (the output stays zero)
    pa, lib, stream, enc = env
    B, Nq, Nkv, Sq, Sk, Hd = 64, 8, 8, 64, 64, 512
    tq = pa.Tensor.empty([B, Nq, Sq, Hd], "f32")
    tk = pa.Tensor.empty([B, Nkv, Sk, Hd], "f32")
    out = pa.Tensor.from_numpy(np.zeros((B, Nq, Sq, Hd), np.float32))
    with pytest.raises(pa.PopcornError) as e:
        _no_alloc(pa, lib, stream, tq, tk, tk, out, B, Nq, Nkv, Sq, Sk, Hd, 0.1, Sk)
    assert e.value.code == -1012
    stream.synchronize()
    assert not out.numpy(stream).any()
