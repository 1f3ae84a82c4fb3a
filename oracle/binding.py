"""ctypes binding of oracle/_build/libpopcorn_oracle.so (test infrastructure).

Every function here forwards to the C restatement in popcorn_oracle.c, which
cites the reference file:line it follows. Arrays are numpy; floating inputs
are float32 (already widened from bf16/f16 where the dtype says so).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

F32, F16, BF16 = 8, 9, 10

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libpopcorn_oracle.so")
_lib = None

_fp = C.POINTER(C.c_float)
_u16p = C.POINTER(C.c_uint16)
_i32p = C.POINTER(C.c_int32)


def build() -> str:
    """Compiles the oracle with its Makefile (gcc, a second or two)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.oracle_xorshift64_next.restype = C.c_uint64
        L.oracle_xorshift64_next.argtypes = [C.POINTER(C.c_uint64)]
        L.oracle_fa_test_float.restype = C.c_float
        L.oracle_fa_test_float.argtypes = [C.POINTER(C.c_uint64)]
        L.oracle_fill_fa_test.argtypes = [C.c_uint64, _fp, C.c_size_t]
        L.oracle_fill_normal.argtypes = [C.c_uint64, C.c_float, C.c_float, _fp, C.c_size_t]
        L.oracle_f32_to_bf16.restype = C.c_uint16
        L.oracle_f32_to_bf16.argtypes = [C.c_float]
        L.oracle_bf16_to_f32.restype = C.c_float
        L.oracle_bf16_to_f32.argtypes = [C.c_uint16]
        L.oracle_f32_to_f16.restype = C.c_uint16
        L.oracle_f32_to_f16.argtypes = [C.c_float]
        L.oracle_f16_to_f32.restype = C.c_float
        L.oracle_f16_to_f32.argtypes = [C.c_uint16]
        L.oracle_convert.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_size_t]
        L.oracle_kv_cache_write.restype = C.c_int
        L.oracle_kv_cache_write.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int] + [C.c_uint32] * 6
        L.oracle_rmsnorm.argtypes = [_fp, _fp, _fp, C.c_size_t, C.c_size_t, C.c_float, C.c_int]
        L.oracle_matmul.argtypes = [_fp, _fp, _fp, C.c_size_t, C.c_size_t, C.c_size_t, C.c_int]
        L.oracle_gelu_tanh_scalar.restype = C.c_float
        L.oracle_gelu_tanh_scalar.argtypes = [C.c_float]
        L.oracle_gelu_tanh.argtypes = [_fp, _fp, C.c_size_t]
        L.oracle_mul.argtypes = [_fp, _fp, _fp, C.c_size_t]
        L.oracle_add.argtypes = [_fp, _fp, _fp, C.c_size_t]
        L.oracle_scalar_mul.argtypes = [_fp, C.c_float, _fp, C.c_size_t]
        L.oracle_gated_mlp.argtypes = [_fp, _fp, C.c_float, C.c_int, _fp, _fp, _fp,
                                       C.c_size_t, C.c_size_t, C.c_int, _fp, _fp]
        L.oracle_attention_naive.argtypes = [_fp, _fp, _fp, _fp] + [C.c_uint32] * 7 + [
            C.c_float, C.c_uint32, C.c_int32]
        L.oracle_flash_decoding.argtypes = [_fp, _fp, _fp, _fp] + [C.c_uint32] * 7 + [
            C.c_float, C.c_uint32, C.c_int32, _fp, _fp, _fp]
        L.oracle_flash_attention_rows.argtypes = [_fp, _fp, _fp, _fp] + [C.c_uint32] * 8 + [
            C.c_float, C.c_uint32, C.c_int32]
        L.oracle_rope_build_cos_sin.argtypes = [_i32p, _fp, _fp, _fp, C.c_uint32, C.c_uint32, C.c_float]
        L.oracle_rope_apply.argtypes = [_fp, _fp, _fp, _fp] + [C.c_uint32] * 4
        L.oracle_transpose12.argtypes = [_fp, _fp] + [C.c_uint32] * 4
        _u32p = C.POINTER(C.c_uint32)
        L.oracle_aq_unpack.restype = C.c_uint32
        L.oracle_aq_unpack.argtypes = [_u32p, C.c_size_t, C.c_int]
        L.oracle_aq_matmul.argtypes = [_fp, _u32p, _fp, _fp, _fp] + [C.c_size_t] * 3 + [C.c_int, C.c_int]
        L.oracle_aq_embedding_gather.argtypes = [_i32p, _u32p, _fp, _fp, _fp, C.c_size_t, C.c_size_t, C.c_int,
                                                 C.c_int]
        L.oracle_argmax.argtypes = [_fp, C.c_size_t, C.c_size_t, _i32p]
        L.oracle_embedding_gather.argtypes = [_i32p, _fp, _fp, C.c_size_t, C.c_size_t]
        L.oracle_decoder_layer.argtypes = [C.c_void_p, _fp, _fp, _fp, C.c_uint32]
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray):
    return a.ctypes.data_as(_fp)


def _np_dtype(tag: int):
    return np.float32 if tag == F32 else np.uint16


# ---- generators -----------------------------------------------------------

def xorshift64_sequence(seed: int, n: int) -> np.ndarray:
    st = C.c_uint64(seed)
    return np.array([lib().oracle_xorshift64_next(C.byref(st)) for _ in range(n)], dtype=np.uint64)


def fa_test_floats(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().oracle_fill_fa_test(seed, _p(out), n)
    return out


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, np.float32)
    lib().oracle_fill_normal(seed, mean, std, _p(out), n)
    return out.reshape(shape)


# ---- conversions ----------------------------------------------------------

def to_bits(x: np.ndarray, tag: int) -> np.ndarray:
    """f32 values -> storage of dtype `tag` (uint16 bits for bf16/f16)."""
    x = _f32(x)
    if tag == F32:
        return x.copy()
    out = np.empty(x.shape, np.uint16)
    lib().oracle_convert(x.ctypes.data, F32, out.ctypes.data, tag, x.size)
    return out


def from_bits(b: np.ndarray, tag: int) -> np.ndarray:
    """storage of dtype `tag` -> f32 values."""
    if tag == F32:
        return _f32(b).copy()
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().oracle_convert(b.ctypes.data, tag, out.ctypes.data, F32, b.size)
    return out


def round_to(x: np.ndarray, tag: int) -> np.ndarray:
    return from_bits(to_bits(x, tag), tag)


# ---- kernels --------------------------------------------------------------

def kv_cache_write(src: np.ndarray, src_tag: int, cache: np.ndarray, cache_tag: int, offset: int) -> int:
    """In-place on `cache` ([B,Nkv,Smax,Hd] storage); returns 0 or a PopcornError code."""
    B, Nkv, Snew, Hd = src.shape
    Smax = cache.shape[2]
    src = np.ascontiguousarray(src)
    assert cache.flags["C_CONTIGUOUS"]
    return lib().oracle_kv_cache_write(src.ctypes.data, src_tag, cache.ctypes.data, cache_tag,
                                       B, Nkv, Snew, Smax, Hd, offset)


def rmsnorm(x: np.ndarray, weight, eps: float, add_one: bool = False) -> np.ndarray:
    x = _f32(x)
    H = x.shape[-1]
    rows = x.size // H
    out = np.empty_like(x)
    w = _f32(weight) if weight is not None else None
    lib().oracle_rmsnorm(_p(x), _p(w) if w is not None else None, _p(out), rows, H, eps, int(add_one))
    return out


def matmul(a: np.ndarray, b: np.ndarray, M: int, K: int, N: int, transpose_b: bool) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    c = np.empty(M * N, np.float32)
    lib().oracle_matmul(_p(a), _p(b), _p(c), M, K, N, int(transpose_b))
    return c.reshape(M, N)


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().oracle_gelu_tanh(_p(x), _p(out), x.size)
    return out


def mul(a, b):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().oracle_mul(_p(a), _p(b), _p(out), a.size)
    return out


def add(a, b):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().oracle_add(_p(a), _p(b), _p(out), a.size)
    return out


def scalar_mul(a, s: float):
    a = _f32(a)
    out = np.empty_like(a)
    lib().oracle_scalar_mul(_p(a), s, _p(out), a.size)
    return out


def gated_mlp(x, norm_w, eps, w_gate, w_up, w_down, inter_tag=F32, add_one=False):
    """Returns (h, out): h the gated intermediate [F], out the down projection [H] (f32)."""
    x, norm_w = _f32(x), _f32(norm_w)
    w_gate, w_up, w_down = _f32(w_gate), _f32(w_up), _f32(w_down)
    F, H = w_gate.shape
    h = np.empty(F, np.float32)
    out = np.empty(H, np.float32)
    lib().oracle_gated_mlp(_p(x), _p(norm_w), eps, int(add_one), _p(w_gate), _p(w_up), _p(w_down),
                           H, F, inter_tag, _p(h), _p(out))
    return h, out


def attention_naive(q, k, v, scale, mask_kind=0, window=-1, key_len=None):
    """q [B,Nq,Sq,Hd]; k,v [B,Nkv,cap,Hd] with key_len (default cap) keys used."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, Nq, Sq, Hd = q.shape
    Nkv, cap = k.shape[1], k.shape[2]
    Sk = cap if key_len is None else key_len
    out = np.empty_like(q)
    lib().oracle_attention_naive(_p(q), _p(k), _p(v), _p(out), B, Nq, Nkv, Sq, Sk, cap, Hd,
                                 scale, mask_kind, window)
    return out


def flash_decoding(q, k, v, scale, P, mask_kind=0, window=-1, key_len=None, return_partials=False):
    """q [B,Nq,1,Hd]; k,v [B,Nkv,cap,Hd]; split into P partitions then combined."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, Nq, Sq, Hd = q.shape
    assert Sq == 1
    Nkv, cap = k.shape[1], k.shape[2]
    Sk = cap if key_len is None else key_len
    out = np.empty_like(q)
    po = np.empty((B, Nq, P, Hd), np.float32)
    pm = np.empty((B, Nq, P), np.float32)
    pl = np.empty((B, Nq, P), np.float32)
    lib().oracle_flash_decoding(_p(q), _p(k), _p(v), _p(out), B, Nq, Nkv, Sk, cap, Hd, P, scale,
                                mask_kind, window, _p(po), _p(pm), _p(pl))
    if return_partials:
        return out, po, pm, pl
    return out


def flash_attention_rows(q, k, v, scale, Bc=128, mask_kind=0, window=-1, key_len=None):
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, Nq, Sq, Hd = q.shape
    Nkv, cap = k.shape[1], k.shape[2]
    Sk = cap if key_len is None else key_len
    out = np.empty_like(q)
    lib().oracle_flash_attention_rows(_p(q), _p(k), _p(v), _p(out), B, Nq, Nkv, Sq, Sk, cap, Hd, Bc,
                                      scale, mask_kind, window)
    return out


def rope_build_cos_sin(positions, inv_freq, scaling=1.0):
    """positions i32 [T], inv_freq [Hd2] -> (cos, sin) f32 [T, Hd2]."""
    pos = np.ascontiguousarray(positions, dtype=np.int32).ravel()
    inv = _f32(inv_freq).ravel()
    T, Hd2 = pos.size, inv.size
    c = np.empty((T, Hd2), np.float32)
    s = np.empty((T, Hd2), np.float32)
    lib().oracle_rope_build_cos_sin(pos.ctypes.data_as(_i32p), _p(inv), _p(c), _p(s), T, Hd2, scaling)
    return c, s


def rope_apply(x, cos, sin):
    """x [B, T, Nh, Hd] with tables [T, Hd/2] -> f32 [B, T, Nh, Hd] (before the output store)."""
    x, cos, sin = _f32(x), _f32(cos), _f32(sin)
    B, T, Nh, Hd = x.shape
    out = np.empty_like(x)
    lib().oracle_rope_apply(_p(x), _p(cos), _p(sin), _p(out), B, T, Nh, Hd // 2)
    return out


def transpose12(src):
    """[D0, D1, D2, D3] -> [D0, D2, D1, D3]."""
    src = _f32(src)
    D0, D1, D2, D3 = src.shape
    out = np.empty((D0, D2, D1, D3), np.float32)
    lib().oracle_transpose12(_p(src), _p(out), D0, D1, D2, D3)
    return out


def _u32(a):
    a = np.ascontiguousarray(a, dtype=np.uint32)
    return a, a.ctypes.data_as(C.POINTER(C.c_uint32))


def aq_unpack(words, count: int, bits: int = 4) -> np.ndarray:
    """Values 0..count-1 of a packed little-endian u32 stream."""
    w, wp = _u32(words)
    return np.array([lib().oracle_aq_unpack(wp, i, bits) for i in range(count)], np.uint32)


def aq_matmul(x, packed, scales, biases, N: int, K: int, bits: int = 4, group: int = 64) -> np.ndarray:
    """x [M, K] f32, packed u32 [N, K*bits/32], scales/biases f32 [N, K/group] -> y [M, N]."""
    x = _f32(x).reshape(-1, K)
    M = x.shape[0]
    w, wp = _u32(packed)
    s = _f32(scales)
    b = _f32(biases) if biases is not None else None
    y = np.empty((M, N), np.float32)
    lib().oracle_aq_matmul(_p(x), wp, _p(s), _p(b) if b is not None else None, _p(y), M, N, K, bits, group)
    return y


def aq_embedding_gather(ids, packed, scales, biases, H: int, bits: int = 4, group: int = 64) -> np.ndarray:
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    w, wp = _u32(packed)
    s = _f32(scales)
    b = _f32(biases) if biases is not None else None
    out = np.empty((ids.size, H), np.float32)
    lib().oracle_aq_embedding_gather(ids.ctypes.data_as(_i32p), wp, _p(s), _p(b) if b is not None else None, _p(out),
                                     ids.size, H, bits, group)
    return out


def argmax(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    N = x.shape[-1]
    rows = x.size // N
    idx = np.empty(rows, np.int32)
    lib().oracle_argmax(_p(x), rows, N, idx.ctypes.data_as(_i32p))
    return idx


def embedding_gather(ids: np.ndarray, table: np.ndarray) -> np.ndarray:
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    table = _f32(table)
    H = table.shape[1]
    out = np.empty((ids.size, H), np.float32)
    lib().oracle_embedding_gather(ids.ctypes.data_as(_i32p), _p(table), _p(out), ids.size, H)
    return out


class _Layer(C.Structure):
    _fields_ = [("H", C.c_uint32), ("Nq", C.c_uint32), ("Nkv", C.c_uint32), ("Hd", C.c_uint32),
                ("F", C.c_uint32), ("kv_capacity", C.c_uint32), ("eps", C.c_float), ("scale", C.c_float),
                ("act_dtype", C.c_int),
                ("w_in_norm", _fp), ("w_qkv", _fp), ("w_o", _fp), ("w_post_attn_norm", _fp),
                ("w_pre_ffn_norm", _fp), ("w_gate", _fp), ("w_up", _fp), ("w_down", _fp),
                ("w_post_ffn_norm", _fp), ("w_q_norm", _fp), ("w_k_norm", _fp), ("v_norm", C.c_int),
                ("inv_freq", _fp), ("rope_scaling", C.c_float)]


def decoder_layer(weights: dict, x: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, pos: int,
                  *, H, Nq, Nkv, Hd, F, eps, scale, act_tag, v_norm=False, rope_scaling=1.0) -> None:
    """In place on x [H], k_cache/v_cache [Nkv, cap, Hd] (f32 storage of act_tag values).
    Optional weights "q_norm", "k_norm" [Hd] and "inv_freq" [Hd/2] (with v_norm) make it a
    real attention block."""
    keep = {n: _f32(w) for n, w in weights.items() if w is not None}
    assert x.dtype == np.float32 and x.flags["C_CONTIGUOUS"]
    cap = k_cache.shape[1]
    opt = [_p(keep[n]) if n in keep else None for n in ("q_norm", "k_norm")]
    L = _Layer(H, Nq, Nkv, Hd, F, cap, eps, scale, act_tag,
               *[_p(keep[n]) for n in ("in_norm", "qkv", "o", "post_attn_norm", "pre_ffn_norm",
                                       "gate", "up", "down", "post_ffn_norm")],
               opt[0], opt[1], int(v_norm), _p(keep["inv_freq"]) if "inv_freq" in keep else None,
               rope_scaling)
    lib().oracle_decoder_layer(C.byref(L), _p(x), _p(k_cache), _p(v_cache), pos)
