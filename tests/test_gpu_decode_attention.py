"""GPU parity of the decode attention block (popcorn_kernel_decode_attention):
raw q/k/v projections -> per-head RMSNorms and RoPE -> new K/V row written to
the caches -> split-KV attention, against the oracle composition of the
reference's dispatches (Gemma4TextInference.swift:352-399: RMSNorm, RopeApply,
Transpose12, KVCacheWrite, FlashAttention), and against the same sequence
run with this library's standalone kernels."""
import numpy as np
import pytest

import oracle as O
from conftest import assert_out
from gpu_util import EPS, download, gpu_env, rounded, upload

pytestmark = pytest.mark.gpu

EPS_NORM = 1e-6


@pytest.fixture(scope="module")
def env():
    return gpu_env()


def _inv_freq(hd, base=10_000.0):
    return np.array([1 / base ** (2 * i / hd) for i in range(hd // 2)], np.float32)


def _oracle_block(qkv, kc, vc, pos, Nq, Nkv, Hd, wq, wk, v_norm, inv, rope_scaling, scale, mask_kind, window, dt):
    """The reference's per-token sequence on the oracle, each stored tensor
    rounded to `dt`; returns the attention output and the processed k, v rows."""
    B = qkv.shape[0]
    r = lambda a: rounded(a, dt)  # noqa: E731
    q = qkv[:, :Nq * Hd].reshape(B, Nq, Hd)
    k = qkv[:, Nq * Hd:(Nq + Nkv) * Hd].reshape(B, Nkv, Hd)
    v = qkv[:, (Nq + Nkv) * Hd:].reshape(B, Nkv, Hd)
    if wq is not None:
        q = r(O.rmsnorm(q, wq, EPS_NORM))
    if wk is not None:
        k = r(O.rmsnorm(k, wk, EPS_NORM))
    if v_norm:
        v = r(O.rmsnorm(v, None, EPS_NORM))
    if inv is not None:
        c, s = O.rope_build_cos_sin([pos], inv, rope_scaling)
        q = r(O.rope_apply(q.reshape(B, 1, Nq, Hd), c, s).reshape(B, Nq, Hd))
        k = r(O.rope_apply(k.reshape(B, 1, Nkv, Hd), c, s).reshape(B, Nkv, Hd))
    kc, vc = kc.copy(), vc.copy()
    kc[:, :, pos] = k
    vc[:, :, pos] = v
    out = O.attention_naive(q.reshape(B, Nq, 1, Hd), kc, vc, scale, mask_kind=mask_kind, window=window,
                            key_len=pos + 1)
    return out, k, v


def _case(env, dt, B, Nq, Nkv, Hd, cap, pos, *, qn=True, kn=True, vn=True, rope=True, scale=None,
          mask_kind=0, window=-1, seed=0, out_dt=None):
    # scale defaults to 1/sqrt(Hd): with unit-variance random heads the logits
    # are then O(1), so the bar measures the arithmetic, not the conditioning
    # of a softmax over logits of size sqrt(Hd) (the reference's Gemma-4 uses
    # scale 1 with trained q/k norm weights that keep its logits in range)
    pa, lib, stream, enc = env
    out_dt = out_dt or dt
    scale = 1 / np.sqrt(Hd) if scale is None else scale
    rng = np.random.default_rng(seed)
    qkv = rounded(rng.standard_normal((B, (Nq + 2 * Nkv) * Hd)).astype(np.float32), dt)
    kc = rounded(rng.standard_normal((B, Nkv, cap, Hd)).astype(np.float32), dt)
    vc = rounded(rng.standard_normal((B, Nkv, cap, Hd)).astype(np.float32), dt)
    wq = (1 + 0.1 * rng.standard_normal(Hd)).astype(np.float32) if qn else None
    wk = (1 + 0.1 * rng.standard_normal(Hd)).astype(np.float32) if kn else None
    inv = _inv_freq(Hd) if rope else None
    tk, tv = upload(pa, kc, dt), upload(pa, vc, dt)
    to = pa.Tensor.empty([B, Nq, 1, Hd], out_dt)
    tpos = pa.Tensor.from_numpy(np.array([pos], np.int32))
    opt = lambda a: upload(pa, a, "f32") if a is not None else None  # noqa: E731
    kern = pa.Kernels.DecodeAttention(upload(pa, qkv, dt), tk, tv, to, tpos, query_heads=Nq, kv_heads=Nkv,
                                      scale=scale, q_norm=opt(wq), k_norm=opt(wk), v_norm=vn, inv_freq=opt(inv),
                                      eps=EPS_NORM, mask=pa.AttentionMask(mask_kind, window))
    enc.encode(kern)
    stream.synchronize()
    ref, kr, vr = _oracle_block(qkv, kc, vc, pos, Nq, Nkv, Hd, wq, wk, vn, inv, 1.0, scale, mask_kind, window, dt)
    what = f"{dt} B={B} Nq={Nq} Nkv={Nkv} Hd={Hd} pos={pos} flags={qn}{kn}{vn}{rope} mask={mask_kind}"
    gk, gv = download(tk, stream), download(tv, stream)
    # every other cache row is untouched, bit for bit
    keep = np.ones(cap, bool)
    keep[pos] = False
    np.testing.assert_array_equal(gk[:, :, keep], kc[:, :, keep], err_msg=what)
    np.testing.assert_array_equal(gv[:, :, keep], vc[:, :, keep], err_msg=what)
    # the new rows: the norm's f32 scale may round one ulp apart, and RoPE
    # rounds once more, so up to two output ulps
    assert_out(gk[:, :, pos], kr, EPS[dt], dt, "k row " + what, half_ulps=4)
    assert_out(gv[:, :, pos], vr, EPS[dt], dt, "v row " + what, half_ulps=4)
    assert_out(download(to, stream), ref, EPS[dt], out_dt, "out " + what, half_ulps=2)
    return kern


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("B,Nq,Nkv,Hd", [(1, 8, 4, 256), (1, 16, 8, 128), (2, 4, 1, 64), (1, 8, 1, 128),
                                         (1, 4, 2, 512), (1, 16, 1, 64)])
def test_decode_attention_vs_oracle(env, dt, B, Nq, Nkv, Hd):
    cap = 1100
    for pos in (0, 1, 63, 64, 777, cap - 1):
        kern = _case(env, dt, B, Nq, Nkv, Hd, cap, pos, seed=pos + Hd)
    assert kern.function_names[0].startswith(f"flash_decoding_fresh_{dt}_l")


@pytest.mark.parametrize("flags", [(False, False, False, False), (True, True, False, False),
                                   (False, False, False, True), (True, False, True, True)])
def test_decode_attention_flag_subsets(env, flags):
    qn, kn, vn, rope = flags
    for pos in (0, 300, 4095):
        _case(env, "bf16", 1, 8, 4, 256, 4352, pos, qn=qn, kn=kn, vn=vn, rope=rope, scale=1 / 16, seed=pos)


def test_decode_attention_f32_and_masks(env):
    _case(env, "f32", 1, 8, 4, 256, 600, 555, seed=1)
    _case(env, "f32", 1, 4, 2, 128, 600, 17, seed=2)
    _case(env, "bf16", 1, 8, 4, 256, 600, 555, out_dt="f32", seed=3)
    _case(env, "bf16", 1, 8, 4, 256, 2000, 1500, mask_kind=1, window=40, seed=4)
    _case(env, "bf16", 1, 8, 4, 256, 2000, 10, mask_kind=1, window=40, seed=5)
    _case(env, "bf16", 1, 8, 4, 256, 2000, 1999, mask_kind=2, seed=6)


def test_decode_attention_matches_standalone_sequence(env):
    # the reference's dispatch sequence with this library's standalone kernels:
    # RMSNorm per head, RopeBuildCosSin + RopeApply (f32 tables), KVCacheWrite,
    # FlashAttention at one query row; same inputs as the fused block
    pa, lib, stream, enc = env
    B, Nq, Nkv, Hd, cap, pos = 1, 8, 4, 256, 4352, 4096
    rng = np.random.default_rng(11)
    qkv = rounded(rng.standard_normal((B, (Nq + 2 * Nkv) * Hd)).astype(np.float32), "bf16")
    kc = rounded(rng.standard_normal((B, Nkv, cap, Hd)).astype(np.float32), "bf16")
    vc = rounded(rng.standard_normal((B, Nkv, cap, Hd)).astype(np.float32), "bf16")
    wq = (1 + 0.1 * rng.standard_normal(Hd)).astype(np.float32)
    wk = (1 + 0.1 * rng.standard_normal(Hd)).astype(np.float32)
    inv = _inv_freq(Hd)
    tq = upload(pa, qkv[:, :Nq * Hd].reshape(1, 1, Nq, Hd), "bf16")
    tkr = upload(pa, qkv[:, Nq * Hd:(Nq + Nkv) * Hd].reshape(1, 1, Nkv, Hd), "bf16")
    tvr = upload(pa, qkv[:, (Nq + Nkv) * Hd:].reshape(1, 1, Nkv, Hd), "bf16")
    tk, tv = upload(pa, kc, "bf16"), upload(pa, vc, "bf16")
    e = lambda shape: pa.Tensor.empty(shape, "bf16")  # noqa: E731
    qn, qr, qa = e([1, 1, Nq, Hd]), e([1, 1, Nq, Hd]), e([1, Nq, 1, Hd])
    kn, kr, ka = e([1, 1, Nkv, Hd]), e([1, 1, Nkv, Hd]), e([1, Nkv, 1, Hd])
    vn, va = e([1, 1, Nkv, Hd]), e([1, Nkv, 1, Hd])
    cos, sin = pa.Tensor.empty([1, Hd // 2], "f32"), pa.Tensor.empty([1, Hd // 2], "f32")
    tpos = pa.Tensor.from_numpy(np.array([pos], np.int32))
    K = pa.Kernels
    seq = [K.RopeBuildCosSin(tpos, upload(pa, inv, "f32"), cos, sin),
           K.RMSNorm(tq, upload(pa, wq, "f32"), qn, eps=EPS_NORM), K.RopeApply(qn, cos, sin, qr), K.Transpose12(qr, qa),
           K.RMSNorm(tkr, upload(pa, wk, "f32"), kn, eps=EPS_NORM), K.RMSNorm(tvr, None, vn, eps=EPS_NORM),
           K.RopeApply(kn, cos, sin, kr), K.Transpose12(kr, ka), K.Transpose12(vn, va),
           K.KVCacheWrite(ka, tk, pos), K.KVCacheWrite(va, tv, pos)]
    out_seq = pa.Tensor.empty([1, Nq, 1, Hd], "bf16")
    seq.append(K.FlashAttention(qa, tk, tv, out=out_seq, scale=1.0, batch=1, query_heads=Nq, kv_heads=Nkv,
                                query_len=1, key_len=pos + 1, head_dim=Hd, key_capacity=cap))
    for k in seq:
        enc.encode(k)
    stream.synchronize()
    k_seq, v_seq, o_seq = download(tk, stream)[:, :, pos], download(tv, stream)[:, :, pos], download(out_seq, stream)

    tk2, tv2 = upload(pa, kc, "bf16"), upload(pa, vc, "bf16")
    out_fused = pa.Tensor.empty([1, Nq, 1, Hd], "bf16")
    enc.encode(K.DecodeAttention(upload(pa, qkv, "bf16"), tk2, tv2, out_fused, tpos, query_heads=Nq, kv_heads=Nkv,
                                 scale=1.0, q_norm=upload(pa, wq, "f32"), k_norm=upload(pa, wk, "f32"), v_norm=True,
                                 inv_freq=upload(pa, inv, "f32"), eps=EPS_NORM))
    stream.synchronize()
    assert_out(download(tk2, stream)[:, :, pos], k_seq, EPS["bf16"], "bf16", "k row fused vs sequence", half_ulps=4)
    assert_out(download(tv2, stream)[:, :, pos], v_seq, EPS["bf16"], "bf16", "v row fused vs sequence", half_ulps=4)
    assert_out(download(out_fused, stream), o_seq, EPS["bf16"], "bf16", "out fused vs sequence", half_ulps=2)
