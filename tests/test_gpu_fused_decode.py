"""GPU parity: the decode matvec with its fused layer glue (residual add of a
post-normed delta, pre-norm, KV-cache scatter) and the gated MLP with its
fused residual, each against the reference's unfused composition in the
oracle (RMSNorm.metal, Add.metal, Matvec.metal, KVCacheWrite.metal, every
intermediate stored in the activation dtype)."""
import numpy as np
import pytest

import oracle as O
import flips
from conftest import assert_out
from flips import assert_any
from gpu_util import EPS, TAG, download, gpu_env, rounded, upload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def assert_residual(actual, x_in, delta, w_post, eps, dtype, bar, what):
    assert_any(actual, flips.residual_candidates(x_in, delta, w_post, eps, TAG[dtype]), bar, dtype, what)


def product_candidates(x, w_pre, w, tag):
    """x W^T for each rounding outcome of the pre-norm (or x itself)."""
    K = x.shape[-1]
    N = w.shape[0]
    vs = flips.norm_candidates(x, w_pre, 1e-6, tag) if w_pre is not None else [x]
    return [O.matmul(v, w, 1, K, N, True).ravel() for v in vs]


@pytest.mark.parametrize("dtype,ot", [("bf16", "bf16"), ("bf16", "f32"), ("f16", "f16"), ("f32", "f32")])
@pytest.mark.parametrize("residual,prenorm", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("K,N", [(2304, 2048), (2048, 2304), (300, 77)])
def test_decode_matvec_glue_vs_composition(env, dtype, ot, residual, prenorm, K, N):
    pa, lib, stream, enc = env
    tag, eps = TAG[dtype], 1e-6
    x_in = rounded(O.normal(K, (K,)), dtype)
    delta = rounded(O.normal(K + 1, (K,), std=3.0), dtype)
    w_post = O.normal(K + 2, (K,), mean=1.0, std=0.1)
    w_pre = O.normal(K + 3, (K,), mean=1.0, std=0.1)
    w = rounded(O.normal(K + 4, (N, K), std=0.02), dtype)
    out = pa.Tensor.empty([N], ot)
    x_out = pa.Tensor.empty([K], dtype)
    kw = {}
    if residual:
        kw.update(delta=upload(pa, delta, dtype), w_post=pa.Tensor.from_numpy(w_post), x_out=x_out)
    if prenorm:
        kw.update(w_pre=pa.Tensor.from_numpy(w_pre))
    k = pa.Kernels.DecodeMatvec(upload(pa, x_in, dtype), upload(pa, w, dtype), out, eps=eps, **kw)
    assert k.function_names[0].startswith(f"decode_matvec_{dtype}_{ot}_r")
    enc.encode(k)
    stream.synchronize()
    bar = 1e-5 if (dtype == "f32") else EPS[dtype]
    x = x_in
    if residual:  # the residual stream first; the product is checked on it
        x = download(x_out, stream)
        assert_residual(x, x_in, delta, w_post, eps, dtype, bar, "residual stream x_out")
    refs = product_candidates(x, w_pre if prenorm else None, w, tag)
    assert_any(download(out, stream), refs, bar, ot, f"decode matvec {dtype}->{ot} r{residual} p{prenorm} {K}x{N}")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("Nq,Nkv,Hd,S,pos", [(8, 4, 256, 64, 17), (8, 1, 256, 4352, 4096), (4, 2, 64, 16, 15)])
def test_decode_matvec_kv_scatter(env, dtype, Nq, Nkv, Hd, S, pos):
    # Gemma QKV projection: rows [0, Nq*Hd) are q, then K rows, then V rows;
    # the K and V rows land in cache[h, pos, :] (KVCacheWrite.metal:1-20 at
    # offset pos) and only q reaches `out`.
    pa, lib, stream, enc = env
    tag, eps = TAG[dtype], 1e-6
    H = 2304 if Hd == 256 else 512
    QW, KW = Nq * Hd, Nkv * Hd
    N = QW + 2 * KW
    x_in = rounded(O.normal(1, (H,)), dtype)
    delta = rounded(O.normal(2, (H,)), dtype)
    w_post = O.normal(3, (H,), mean=1.0, std=0.1)
    w_pre = O.normal(4, (H,), mean=1.0, std=0.1)
    w = rounded(O.normal(5, (N, H), std=0.02), dtype)
    kc0 = rounded(O.normal(6, (Nkv, S, Hd)), dtype)
    vc0 = rounded(O.normal(7, (Nkv, S, Hd)), dtype)
    kc, vc = upload(pa, kc0, dtype), upload(pa, vc0, dtype)
    q = pa.Tensor.empty([QW], dtype)
    x_out = pa.Tensor.empty([H], dtype)
    position = pa.Tensor.from_numpy(np.array([pos], np.int32))
    k = pa.Kernels.DecodeMatvec(upload(pa, x_in, dtype), upload(pa, w, dtype), q, delta=upload(pa, delta, dtype),
                                w_post=pa.Tensor.from_numpy(w_post), x_out=x_out,
                                w_pre=pa.Tensor.from_numpy(w_pre), k_cache=kc, v_cache=vc, position=position,
                                q_rows=QW, eps=eps)
    enc.encode(k)
    stream.synchronize()
    bar = EPS[dtype]
    x = download(x_out, stream)
    assert_residual(x, x_in, delta, w_post, eps, dtype, bar, "residual stream x_out")
    kg, vg = download(kc, stream).reshape(Nkv, S, Hd), download(vc, stream).reshape(Nkv, S, Hd)
    # q, then the K and V rows at pos, in projection row order
    got = np.concatenate([download(q, stream).ravel(), kg[:, pos, :].ravel(), vg[:, pos, :].ravel()])
    assert_any(got, product_candidates(x, w_pre, w, tag), bar, dtype, "q rows + k, v rows at pos")
    others = np.ones(S, bool)
    others[pos] = False
    # every other cache row is untouched, bit for bit
    np.testing.assert_array_equal(O.to_bits(kg[:, others], tag), O.to_bits(kc0[:, others], tag))
    np.testing.assert_array_equal(O.to_bits(vg[:, others], tag), O.to_bits(vc0[:, others], tag))


def test_decode_matvec_scatter_position_out_of_range_writes_nothing(env):
    # a device position outside the cache skips the scatter (the kernel's own
    # bounds check) and leaves both caches as they were
    pa, lib, stream, enc = env
    Nq, Nkv, Hd, S, H = 2, 1, 64, 8, 128
    N = Nq * Hd + 2 * Nkv * Hd
    kc0 = rounded(O.normal(1, (Nkv, S, Hd)), "bf16")
    kc, vc = upload(pa, kc0, "bf16"), upload(pa, kc0, "bf16")
    q = pa.Tensor.empty([Nq * Hd], "bf16")
    for bad in (S, -1):
        k = pa.Kernels.DecodeMatvec(upload(pa, rounded(O.normal(2, (H,)), "bf16"), "bf16"),
                                    upload(pa, rounded(O.normal(3, (N, H), std=0.02), "bf16"), "bf16"), q,
                                    k_cache=kc, v_cache=vc, position=pa.Tensor.from_numpy(np.array([bad], np.int32)),
                                    q_rows=Nq * Hd)
        enc.encode(k)
        stream.synchronize()
        np.testing.assert_array_equal(O.to_bits(download(kc, stream).reshape(kc0.shape), O.BF16),
                                      O.to_bits(kc0, O.BF16))
        np.testing.assert_array_equal(O.to_bits(download(vc, stream).reshape(kc0.shape), O.BF16),
                                      O.to_bits(kc0, O.BF16))


@pytest.mark.parametrize("dtype,H,F", [("bf16", 2304, 9216), ("f16", 512, 2048), ("f32", 256, 1024)])
def test_gated_mlp_residual_vs_composition(env, dtype, H, F):
    # x = x_in + RMSNorm(attn_o) * w_post_attn; mlp = GatedMLP(x)
    # (Gemma4TextInference.swift:398-429 with the post-attention norm folded in)
    pa, lib, stream, enc = env
    tag, eps = TAG[dtype], 1e-6
    x_in = rounded(O.normal(20, (H,)), dtype)
    delta = rounded(O.normal(21, (H,), std=2.0), dtype)
    w_post = O.normal(22, (H,), mean=1.0, std=0.1)
    nw = O.normal(23, (H,), mean=1.0, std=0.1)
    wg, wu = (rounded(O.normal(s, (F, H), std=0.02), dtype) for s in (24, 25))
    wd = rounded(O.normal(26, (H, F), std=0.02), dtype)
    x_out, out = pa.Tensor.empty([H], dtype), pa.Tensor.empty([H], dtype)
    k = pa.Kernels.GatedMLPResidual(upload(pa, x_in, dtype), upload(pa, delta, dtype), pa.Tensor.from_numpy(w_post),
                                    x_out, pa.Tensor.from_numpy(nw), upload(pa, wg, dtype), upload(pa, wu, dtype),
                                    upload(pa, wd, dtype), out, eps=eps)
    enc.encode(k)
    stream.synchronize()
    bar = 1e-5 if dtype == "f32" else EPS[dtype]
    x = download(x_out, stream)
    assert_residual(x, x_in, delta, w_post, eps, dtype, bar, "residual stream")
    # the MLP half is checked on the residual stream the kernel produced (just
    # checked above), over the rounding outcomes of its pre-norm: one midpoint
    # flip in the normed vector shifts every gate and up sum and flips ~10% of
    # the 16-bit hidden roundings, which the down projection sums up
    refs = [flips.mlp_from_normed(n, wg, wu, wd, tag)[1] for n in flips.norm_candidates(x, nw, eps, tag)]
    assert_any(download(out, stream), refs, bar, dtype, "gated MLP (residual) out")
