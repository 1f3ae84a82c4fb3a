"""GPU parity: Matmul (m == 1 matvec and the general fallback), the elementwise
pieces of the gated MLP, and the fused gated MLP, through the C ABI."""
import numpy as np
import pytest

import oracle as O
import flips
from conftest import assert_approx, assert_out, half_ulp
from flips import assert_any
from gpu_util import EPS, TAG, download, gpu_env, rounded, upload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def _run(env, kernel):
    pa, lib, stream, enc = env
    enc.encode(kernel)
    stream.synchronize()


def test_matmul_reference_kats(env):
    pa, lib, stream, enc = env
    a = pa.Tensor.from_numpy(np.array([1, 2, 3, 4, 5, 6], np.float32).reshape(2, 3))
    b = pa.Tensor.from_numpy(np.array([7, 8, 9, 10, 11, 12], np.float32).reshape(3, 2))
    bt = pa.Tensor.from_numpy(np.array([7, 9, 11, 8, 10, 12], np.float32).reshape(2, 3))
    c1, c2 = pa.Tensor.empty([2, 2]), pa.Tensor.empty([2, 2])
    x = pa.Tensor.from_numpy(np.array([[1, 2, 3]], np.float32))
    y = pa.Tensor.empty([1, 2])
    # KernelsTests.swift:179-190, :217-229, :192-199
    enc.encode(pa.Kernels.Matmul(a, b, c1), pa.Kernels.Matmul(a, bt, c2, True),
               pa.Kernels.Matmul(x, bt, y, True))
    stream.synchronize()
    assert c1.numpy(stream).ravel().tolist() == [58, 64, 139, 154]
    assert c2.numpy(stream).ravel().tolist() == [58, 64, 139, 154]
    assert y.numpy(stream).ravel().tolist() == [58, 64]
    assert pa.Kernels.Matmul(x, bt, y, True).function_names == ["matvec_nk_stream_f32_f32_f32_r1"]


TRIPLES = [("f32", "f32", "f32"), ("f32", "bf16", "f32"), ("bf16", "bf16", "f32"), ("bf16", "bf16", "bf16"),
           ("f32", "f16", "f32"), ("f16", "f16", "f32"), ("f16", "f16", "f16")]


@pytest.mark.parametrize("xt,wt,ot", TRIPLES)
@pytest.mark.parametrize("K,N", [(256, 67), (131, 64), (2304, 9216), (9216, 2304), (2304, 4096), (64, 3)])
def test_matvec_nk_vs_oracle(env, xt, wt, ot, K, N):
    # shapes of KernelsTests.swift:204-215 (vec4 body with N % 4 != 0, K tail)
    # and the Gemma decode projections; W is [N, K] (transposeB)
    pa, lib, stream, enc = env
    x = rounded(O.normal(K + N, (1, K)), xt)
    w = rounded(O.normal(K * 3 + N, (N, K), std=0.02), wt)
    tx, tw = upload(pa, x, xt), upload(pa, w, wt)
    out = pa.Tensor.empty([1, N], ot)
    _run(env, pa.Kernels.Matmul(tx, tw, out, True))
    ref = O.matmul(x, w, 1, K, N, True)
    # inputs are exact in their dtypes and accumulation is f32: an f32 output
    # differs from the oracle only by summation order (1e-5); a 16-bit output
    # adds its store's rounding
    eps = 1e-5 if ot == "f32" else EPS[ot]
    assert_out(download(out, stream), ref, eps, ot, f"matvec {xt},{wt},{ot} K={K} N={N}")


@pytest.mark.parametrize("xt,wt,ot", [("f32", "f32", "f32"), ("bf16", "bf16", "bf16"), ("f32", "bf16", "f32")])
def test_matvec_kn_vs_oracle(env, xt, wt, ot):
    # transposeW == 0 fallback (Matvec.metal:6-30): W is [K, N]
    pa, lib, stream, enc = env
    K, N = 300, 517
    x = rounded(O.normal(1, (1, K)), xt)
    w = rounded(O.normal(2, (K, N), std=0.05), wt)
    out = pa.Tensor.empty([1, N], ot)
    _run(env, pa.Kernels.Matmul(upload(pa, x, xt), upload(pa, w, wt), out, False))
    assert_out(download(out, stream), O.matmul(x, w, 1, K, N, False), 1e-5 if ot == "f32" else 2e-3, ot, "matvec kn")


@pytest.mark.parametrize("M,K,N,tb", [(64, 64, 64, False), (70, 33, 50, False), (64, 64, 64, True), (130, 200, 90, True)])
@pytest.mark.parametrize("at,bt,ot", [("f32", "f32", "f32"), ("bf16", "bf16", "f32"), ("f16", "f16", "f16")])
def test_matmul_general_vs_oracle(env, M, K, N, tb, at, bt, ot):
    # KernelsTests.swift:278-294 shapes, inputs uniform(-1, 1) like runMatmul
    pa, lib, stream, enc = env
    rng = np.random.default_rng(M * K + N)
    a = rounded(rng.uniform(-1, 1, (M, K)), at)
    b = rounded(rng.uniform(-1, 1, (N, K) if tb else (K, N)), bt)
    out = pa.Tensor.empty([M, N], ot)
    _run(env, pa.Kernels.Matmul(upload(pa, a, at), upload(pa, b, bt), out, tb))
    assert_out(download(out, stream), O.matmul(a, b, M, K, N, tb), 1e-5 if ot == "f32" else 2e-3, ot, "matmul")


def test_matmul_integer_exact(env):
    pa, lib, stream, enc = env
    rng = np.random.default_rng(5)
    a = rng.integers(-8, 9, (1, 1024)).astype(np.float32)
    w = rng.integers(-8, 9, (333, 1024)).astype(np.float32)
    out = pa.Tensor.empty([1, 333])
    _run(env, pa.Kernels.Matmul(upload(pa, a, "bf16"), upload(pa, w, "bf16"), out, True))
    np.testing.assert_array_equal(out.numpy(stream).ravel(), (a.astype(np.int64) @ w.T.astype(np.int64)).ravel())


# ---- elementwise --------------------------------------------------------------

def test_elementwise_reference_kats(env):
    pa, lib, stream, enc = env
    x = pa.Tensor.from_numpy(np.array([0, 1, -1, 2], np.float32))
    g = pa.Tensor.empty([4])
    a = pa.Tensor.from_numpy(np.array([1, 2, 3, 4], np.float32))
    b = pa.Tensor.from_numpy(np.array([5, -1, 0.5, 2], np.float32))
    m, s = pa.Tensor.empty([4]), pa.Tensor.empty([4])
    sm = pa.Tensor.empty([4])
    enc.encode(pa.Kernels.GeluTanh(x, g), pa.Kernels.Mul(a, b, m), pa.Kernels.Add(a, b, s),
               pa.Kernels.ScalarMul(pa.Tensor.from_numpy(np.array([1, 2, -3, 4], np.float32)), 2.5, sm))
    stream.synchronize()
    assert_approx(g.numpy(stream), [0.0, 0.8411920, -0.1588080, 1.9545977], 1e-4, "gelu kat")  # :106-117
    assert m.numpy(stream).tolist() == [5, -2, 1.5, 8]  # :88-95
    assert s.numpy(stream).tolist() == [6, 1, 3.5, 6]
    assert sm.numpy(stream).tolist() == [2.5, 5.0, -7.5, 10.0]  # :78-84


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("n", [1, 7, 9216, 100003])
def test_elementwise_vs_oracle(env, dtype, n):
    pa, lib, stream, enc = env
    a = rounded(O.normal(n, (n,), std=3.0), dtype)
    b = rounded(O.normal(n + 1, (n,)), dtype)
    ta, tb = upload(pa, a, dtype), upload(pa, b, dtype)
    g, m, s = (pa.Tensor.empty([n], dtype) for _ in range(3))
    enc.encode(pa.Kernels.GeluTanh(ta, g), pa.Kernels.Mul(ta, tb, m), pa.Kernels.Add(ta, tb, s))
    stream.synchronize()
    eps = 1e-5 if dtype == "f32" else 2e-3
    assert_out(download(g, stream), O.gelu_tanh(a), eps, dtype, "gelu")
    assert_out(download(m, stream), O.mul(a, b), eps, dtype, "mul")
    assert_out(download(s, stream), O.add(a, b), eps, dtype, "add")


# ---- gated MLP -----------------------------------------------------------------

@pytest.mark.parametrize("dtype,H,F", [("bf16", 2304, 9216), ("f32", 256, 1024), ("f16", 3072, 1024), ("bf16", 100, 300)])
def test_gated_mlp_vs_composition(env, dtype, H, F):
    # BASELINE config 3 at full size (bf16 2304 x 9216): RMSNorm w = 1 + N(0, .1),
    # eps 1e-6, weights N(0, .02); parity target is the reference composition
    # with every intermediate stored in the activation dtype.
    pa, lib, stream, enc = env
    x = rounded(O.normal(0, (H,)), dtype)
    nw = O.normal(1, (H,), mean=1.0, std=0.1)
    wg = rounded(O.normal(2, (F, H), std=0.02), dtype)
    wu = rounded(O.normal(3, (F, H), std=0.02), dtype)
    wd = rounded(O.normal(4, (H, F), std=0.02), dtype)
    out = pa.Tensor.empty([H], dtype)
    hid = pa.Tensor.empty([F], dtype)
    k = pa.Kernels.GatedMLP(upload(pa, x, dtype), pa.Tensor.from_numpy(nw), upload(pa, wg, dtype),
                            upload(pa, wu, dtype), upload(pa, wd, dtype), out, eps=1e-6, hidden=hid)
    _run(env, k)
    eps = EPS[dtype]
    # The normalised x is stored in the activation dtype too: the kernel's f32
    # norm scale (its sum of squares in another order) may round an element
    # that sits on a 16-bit midpoint the other way, and since every g and u is
    # a dot product with that vector, ~10% of their roundings then flip. The
    # output and h are held to their bars against the composition on one of
    # the normed vectors a scale within f32 noise yields (flips.py).
    outs = [flips.mlp_from_normed(n, wg, wu, wd, TAG[dtype]) for n in flips.norm_candidates(x, nw, 1e-6, TAG[dtype])]
    assert_any(download(out, stream), [o for _, o in outs], eps, dtype, "gated MLP out")
    # h = round(round(gelu(g)) * u) with g, u rounded too: exactly one of the
    # values the composition yields for the roundings of g, u and gelu(g)
    # that their f32 summation order and the GELU's last bits allow
    # (flips.HiddenOutcomes), on one of the normed vectors
    h = download(hid, stream)
    if dtype == "f32":
        assert_approx(h, outs[0][0], 1e-5, "gated hidden")
    else:
        errors = []
        for n in flips.norm_candidates(x, nw, 1e-6, TAG[dtype]):
            try:
                flips.dense_hidden(n, wg, wu, TAG[dtype]).check(h, "gated hidden")
                break
            except AssertionError as e:
                errors.append(str(e))
        else:
            raise AssertionError(" | ".join(errors))


def test_gated_mlp_scratch_hidden_and_add_one(env):
    pa, lib, stream, enc = env
    H, F = 512, 2048
    x = rounded(O.normal(10, (1, H)), "bf16")
    nw = O.normal(11, (H,), std=0.1)
    wg, wu = (rounded(O.normal(s, (F, H), std=0.02), "bf16") for s in (12, 13))
    wd = rounded(O.normal(14, (H, F), std=0.02), "bf16")
    out = pa.Tensor.empty([1, H], "bf16")
    k = pa.Kernels.GatedMLP(upload(pa, x, "bf16"), pa.Tensor.from_numpy(nw), upload(pa, wg, "bf16"),
                            upload(pa, wu, "bf16"), upload(pa, wd, "bf16"), out, eps=1e-6, add_one_to_weight=True)
    assert k.function_names[0].startswith("gated_mlp_gate_up_bf16")
    _run(env, k)
    refs = [flips.mlp_from_normed(n, wg, wu, wd, O.BF16)[1] for n in flips.norm_candidates(x.ravel(), nw, 1e-6, O.BF16, True)]
    assert_any(download(out, stream).ravel(), refs, 2e-3, "bf16", "gated MLP addOne")
