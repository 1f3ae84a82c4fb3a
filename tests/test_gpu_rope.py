"""GPU parity of the RoPE tables, RoPE and the head transpose
(RopeBuildCosSin.metal, RopeApply.metal, Transpose12.metal) against the
oracle, through the C ABI."""
import numpy as np
import pytest

import oracle as O
from conftest import assert_approx, assert_out
from gpu_util import EPS, download, gpu_env, rounded, upload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def _run(env, k):
    pa, lib, stream, enc = env
    enc.encode(k)
    stream.synchronize()


def _inv_freq(hd, base=10_000.0):
    return np.array([1 / base ** (2 * i / hd) for i in range(hd // 2)], np.float32)


def _tables(env, pos, inv, scaling=1.0):
    pa, lib, stream, enc = env
    T, H2 = len(pos), len(inv)
    tc, ts = pa.Tensor.empty([T, H2], "f32"), pa.Tensor.empty([T, H2], "f32")
    tp = pa.Tensor.from_numpy(np.asarray(pos, np.int32), "i32")
    ti = pa.Tensor.from_numpy(np.asarray(inv, np.float32), "f32")
    k = pa.Kernels.RopeBuildCosSin(tp, ti, tc, ts, attention_scaling=scaling)
    assert k.function_names == ["rope_build_cos_sin"]
    _run(env, k)
    return tc, ts


def test_rope_reference_kat(env):
    # KernelsTests.swift:438-489: positions [0, 1], inv_freq [1, 0.5], x = 1..8
    pa, lib, stream, enc = env
    tc, ts = _tables(env, [0, 1], [1.0, 0.5])
    c, s = download(tc, stream).ravel(), download(ts, stream).ravel()
    f = np.float32
    assert_approx(c, [1, 1, np.cos(f(1)), np.cos(f(0.5))], 1e-4, "cos")
    assert_approx(s, [0, 0, np.sin(f(1)), np.sin(f(0.5))], 1e-4, "sin")
    x = upload(pa, np.arange(1, 9, dtype=np.float32).reshape(1, 2, 1, 4), "f32")
    out = pa.Tensor.empty([1, 2, 1, 4], "f32")
    _run(env, pa.Kernels.RopeApply(x, tc, ts, out, batch=1, seq_len=2, head_count=1, head_dim=4))
    r = download(out, stream).ravel()
    c0, s0, c1, s1 = np.cos(1.0), np.sin(1.0), np.cos(0.5), np.sin(0.5)
    assert_approx(r, [1, 2, 3, 4, 5 * c0 - 7 * s0, 6 * c1 - 8 * s1, 5 * s0 + 7 * c0, 6 * s1 + 8 * c1], 1e-4, "apply")


@pytest.mark.parametrize("scaling", [1.0, 0.5])
def test_rope_tables_vs_oracle(env, scaling):
    pa, lib, stream, enc = env
    pos = np.array([0, 1, 2, 100, 4095, 4096, 32767, 131071, 1 << 20], np.int32)
    for hd, base in ((256, 10_000.0), (512, 1_000_000.0)):
        inv = _inv_freq(hd, base)
        if hd == 512:
            inv[hd // 8:] = 0  # partial rotary of the full-attention layers (Gemma4Workspace.swift:198-201)
        tc, ts = _tables(env, pos, inv, scaling)
        rc, rs = O.rope_build_cos_sin(pos, inv, scaling)
        # f32 outputs at the 1e-5 bar; the library sincos is within a few ulp
        assert_approx(download(tc, stream), rc, EPS["f32"], f"cos hd={hd}")
        assert_approx(download(ts, stream), rs, EPS["f32"], f"sin hd={hd}")


@pytest.mark.parametrize("xt,tt", [("f32", "f32"), ("bf16", "bf16"), ("bf16", "f32")])
@pytest.mark.parametrize("B,T,Nh,Hd", [(1, 1, 8, 256), (2, 7, 4, 128), (1, 33, 3, 64), (1, 5, 2, 20), (1, 3, 1, 2)])
def test_rope_apply_vs_oracle(env, xt, tt, B, T, Nh, Hd):
    pa, lib, stream, enc = env
    rng = np.random.default_rng(B * 1000 + T * 10 + Hd)
    pos = rng.integers(0, 8192, T).astype(np.int32)
    rc, rs = O.rope_build_cos_sin(pos, _inv_freq(Hd))
    c, s = rounded(rc, tt), rounded(rs, tt)
    x = rounded(rng.standard_normal((B, T, Nh, Hd)).astype(np.float32), xt)
    out = pa.Tensor.empty([B, T, Nh, Hd], xt)
    k = pa.Kernels.RopeApply(upload(pa, x, xt), upload(pa, c, tt), upload(pa, s, tt), out)
    _run(env, k)
    ref = O.rope_apply(x, c, s)
    assert_out(download(out, stream), ref, EPS[xt], xt, f"rope {xt}/{tt} {B}x{T}x{Nh}x{Hd}")


def test_rope_apply_unaligned_and_in_place(env):
    # a view starting 2 bytes into its buffer takes the element-by-element
    # path; out == x works (each work item reads its pairs before writing)
    pa, lib, stream, enc = env
    T, Nh, Hd = 3, 2, 64
    rng = np.random.default_rng(5)
    rc, rs = O.rope_build_cos_sin(np.arange(T, dtype=np.int32) * 37, _inv_freq(Hd))
    c, s = rounded(rc, "bf16"), rounded(rs, "bf16")
    x = rounded(rng.standard_normal((1, T, Nh, Hd)).astype(np.float32), "bf16")
    base = upload(pa, np.concatenate([[0.0], x.ravel()]).astype(np.float32), "bf16")
    view = pa.Tensor(base.ptr + 2, [1, T, Nh, Hd], "bf16")
    _run(env, pa.Kernels.RopeApply(view, upload(pa, c, "bf16"), upload(pa, s, "bf16"), view))
    got = download(base, stream)[1:].reshape(1, T, Nh, Hd)
    assert_out(got, O.rope_apply(x, c, s), EPS["bf16"], "bf16", "rope unaligned in place")


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("shape", [(1, 2, 8, 256), (2, 9, 3, 128), (1, 5, 4, 7), (3, 1, 6, 8), (1, 2048, 16, 256)])
def test_transpose12_bit_exact(env, dt, shape):
    pa, lib, stream, enc = env
    rng = np.random.default_rng(sum(shape))
    x = rounded(rng.standard_normal(shape).astype(np.float32), dt)
    src = upload(pa, x, dt)
    out = pa.Tensor.empty([shape[0], shape[2], shape[1], shape[3]], dt)
    k = pa.Kernels.Transpose12(src, out)
    assert k.function_names == [{"f32": "transpose12", "f16": "transpose12_f16", "bf16": "transpose12_bf16"}[dt]]
    _run(env, k)
    np.testing.assert_array_equal(download(out, stream), O.transpose12(x))
