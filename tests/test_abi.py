"""CPU tests of the C ABI: the library loads, exports every function that
include/*.h declares, and the descriptors validate and route without a GPU
(fake device addresses: nothing is launched)."""
import glob
import json
import os
import re

import pytest

import popcorn_amd as pa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE = 0x7F0000000000  # never dereferenced: descriptors only validate


def declared_functions():
    names = set()
    inc = os.path.join(ROOT, "include")
    for f in os.listdir(inc):
        if f.endswith(".h"):
            text = open(os.path.join(inc, f)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(popcorn_[a-z0-9_]+)\s*\(", text))
    return sorted(n for n in names if not n.endswith("_t"))  # types in function-pointer fields


def test_every_declared_symbol_is_exported():
    lib = pa.lib()
    names = declared_functions()
    assert len(names) > 50
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_bindings_cover_the_header():
    from popcorn_amd._capi import PROTOTYPES

    assert set(declared_functions()) <= set(PROTOTYPES)


def T(shape, dtype="bf16", ptr=FAKE):
    return pa.Tensor(ptr, shape, dtype)


def test_dtype_stride_and_scratch_spec():
    # Tensor.swift:152-159, ScratchSpec.swift / KernelResourceTests.swift:5-8
    assert [pa.stride(d) for d in ("u8", "bf16", "f16", "f32", "i32", "i64")] == [1, 2, 2, 4, 4, 8]
    assert pa.scratch_spec_byte_count([2, 3, 4], "f32") == 96
    assert pa.scratch_spec_byte_count([], "bf16") == 2


def test_status_mapping():
    lib = pa.lib()
    assert lib.popcorn_status_from_hip_error(0) == 0
    assert lib.popcorn_status_from_hip_error(2) == -1013   # out of memory
    assert lib.popcorn_status_from_hip_error(702) == -1014  # launch timeout
    assert lib.popcorn_status_from_hip_error(700) == -1015  # illegal address
    assert lib.popcorn_status_from_hip_error(400) == -1016  # invalid handle
    assert lib.popcorn_status_from_hip_error(100) == -1017  # no device
    assert lib.popcorn_status_from_hip_error(999) == -1019


def test_route():
    # FlashAttention.swift:109-113
    assert pa.Kernels.route(1, 256) == "decoding"
    assert pa.Kernels.route(2, 256) == "plain"


def test_prefill_attention_head_dims():
    # Sq >= 32 and any 16-bit head dim up to 512 in 16-byte rows take the
    # matrix cores (the reference's MPP route, FlashAttention.swift:109-113,
    # hd256/hd512 buckets :305-311), padded to the kernel's 64/128/256/512
    def fa(Hd, S=640, dtype="bf16", out=None):
        q = T([1, 2, S, Hd], dtype)
        return pa.Kernels.FlashAttention(q, q, q, out=T([1, 2, S, Hd], out or dtype), scale=0.1,
                                         batch=1, query_heads=2, kv_heads=2, query_len=S, key_len=S,
                                         head_dim=Hd).function_names
    assert fa(512) == ["flash_attention_tiled16_bf16_bf16_d512"]          # whole tiles, no merge
    assert fa(512, S=4096) == ["flash_attention_tiled16_bf16_bf16_d512"]
    assert fa(512, out="f32") == ["flash_attention_tiled16_bf16_f32_d512"]
    assert fa(320, dtype="f16") == ["flash_attention_tiled16_f16_f16_d512"]
    assert fa(192) == ["flash_attention_tiled16_bf16_bf16_d256"]
    assert fa(80) == ["flash_attention_tiled16_bf16_bf16_d128"]
    assert fa(40) == ["flash_attention_tiled_bf16_bf16_d64"]
    assert fa(8) == ["flash_attention_tiled_bf16_bf16_d64"]
    assert fa(36)[0].startswith("flash_decoding_partial_")   # not 16-byte rows: the per-row kernel


def test_prefill_attention_split_plan():
    # causal prefill with at most two 128-row tiles per CU (256 CUs when no
    # GPU answers). At most one tile per CU: light and heavy tiles paired,
    # the second block of a pair merging the split tile itself. Up to two
    # per CU: tiles with more than half the last tile's key steps run as two
    # blocks, merged by a second kernel.
    def fa(Nq, S, mask=(0, -1), dtype="f16"):
        q = T([1, Nq, S, 256], dtype)
        return pa.Kernels.FlashAttention(q, q, q, out=T([1, Nq, S, 256], dtype), scale=1 / 16,
                                         mask=pa.AttentionMask(*mask), batch=1, query_heads=Nq, kv_heads=Nq,
                                         query_len=S, key_len=S, head_dim=256).function_names
    assert fa(16, 2048) == ["flash_attention_tiled16_f16_f16_d256"]
    assert fa(16, 2048, dtype="bf16") == ["flash_attention_tiled16_bf16_bf16_d256"]
    assert fa(24, 2048) == ["flash_attention_tiled16_f16_f16_d256", "flash_attention_split_merge_f16_d256"]
    assert fa(16, 2048, mask=(2, -1)) == ["flash_attention_tiled16_f16_f16_d256"]   # every tile sees every key
    assert fa(16, 2048, mask=(1, 256)) == ["flash_attention_tiled16_f16_f16_d256"]  # window: equal work per tile
    assert fa(16, 384) == ["flash_attention_tiled16_f16_f16_d256"]                  # 3 tiles per head
    assert fa(64, 2048) == ["flash_attention_tiled16_f16_f16_d256"]                 # 1024 tiles: 4 per CU


def test_prefill_gemm_tile_plan():
    # MFMA GEMM tiles by CU fill (256 CUs when no GPU answers); a grid of
    # 256 x 384 tiles too small for the CUs splits K into whole rounds
    def mm(M, K, N, dtype="f16", out=None):
        return pa.Kernels.Matmul(T([M, K], dtype), T([N, K], dtype), T([M, N], out or dtype), True).function_names
    # K % 64 == 0: the whole-line ("e") forms; K % 64 == 32: the 64-byte-row ("d") ones
    # whole-line tiles by score (grid fill x inside share x tile throughput)
    assert mm(2048, 3072, 9216) == ["matmul_mfma_f16_f16_f16_e256x288"]    # QKV: 256 tiles of 256 x 288
    assert mm(2048, 3072, 24576) == ["matmul_mfma_f16_f16_f16_e256x384"]   # gate / up: 512 tiles
    assert mm(2048, 3104, 24576) == ["matmul_mfma_f16_f16_f16_d256x384"]   # K % 64 == 32
    assert mm(2048, 24576, 3072) == ["matmul_mfma_f16_splitk_e256x384", "matmul_splitk_reduce_f16"]  # down: 64 x 4
    assert mm(2000, 16384, 1500, "bf16", "f32") == ["matmul_mfma_bf16_splitk_e256x384",
                                                    "matmul_splitk_reduce_f32"]  # 32 tiles x 8 splits
    assert mm(2000, 16640, 1500, "bf16", "f32") == ["matmul_mfma_bf16_splitk_d256x384",
                                                    "matmul_splitk_reduce_f32"]  # splits of 2080: K % 64 == 32
    assert mm(2048, 4096, 3072) == ["matmul_mfma_f16_f16_f16_e128x128"]    # splits would be under 2048 deep
    assert mm(4096, 4096, 3072) == ["matmul_mfma_f16_f16_f16_e128x192"]    # 2 splits of 2048: partials cost more than the tiles lose
    assert mm(4096, 24576, 3072) == ["matmul_mfma_f16_splitk_e256x384", "matmul_splitk_reduce_f16"]  # 128 tiles x 2
    # the split-K reduction stores 4 results at a time: a C not 16-byte aligned keeps one pass
    c_off = pa.Kernels.Matmul(T([2048, 24576], "f16"), T([3072, 24576], "f16"), T([2048, 3072], "f16", FAKE + 8),
                              True).function_names
    assert c_off == ["matmul_mfma_f16_f16_f16_e128x128"]
    assert mm(256, 1024, 384) == ["matmul_mfma_f16_f16_f16_e128x128"]
    assert mm(256, 1056, 384) == ["matmul_mfma_f16_f16_f16_d128x128"]
    # 2 <= M <= 64: the skinny kernel, M padded to 16 per MFMA tile
    assert mm(2, 64, 67) == ["matmul_skinny_f16_f16_f16_m16_r16"]           # 16-row blocks below 256 x 32 rows
    assert mm(8, 9216, 2304, "bf16") == ["matmul_skinny_bf16_bf16_bf16_m16_r16"]
    assert mm(32, 2304, 8160) == ["matmul_skinny_f16_f16_f16_m32_r16"]     # 255 blocks of 32 rows
    assert mm(32, 2304, 8176) == ["matmul_skinny_f16_f16_f16_m32"]         # 256 of 32, 511 tiles of 16
    assert mm(32, 2304, 8192) == ["matmul_skinny_f16_f16_f16_m32_lds"]     # 512 tiles of 16
    # at least 512 tiles of 16 rows of B: A staged in LDS
    assert mm(8, 2304, 9216, "bf16") == ["matmul_skinny_bf16_bf16_bf16_m16_lds"]
    assert mm(17, 2304, 9216, "bf16", "f32") == ["matmul_skinny_bf16_bf16_f32_m32_lds"]
    assert mm(48, 2304, 9216) == ["matmul_skinny_f16_f16_f16_m48_lds"]
    assert mm(64, 3072, 24576) == ["matmul_skinny_f16_f16_f16_m64_lds"]
    assert mm(65, 2048, 2048) == ["matmul_mfma_f16_f16_f16_e128x128"]
    assert mm(8, 2300, 9216)[0].startswith("matmul_tiled")  # K % 8 != 0: the SIMT tiles


def test_flash_attention_routing_names():
    q, o = T([1, 8, 1, 256]), T([1, 8, 1, 256])
    k = T([1, 4, 4352, 256])
    kern = pa.Kernels.FlashAttention(q, k, k, out=o, scale=1 / 16, batch=1, query_heads=8, kv_heads=4,
                                     query_len=1, key_len=4097, head_dim=256, key_capacity=4352)
    assert kern.function_names == ["flash_decoding_partial_bf16_l32_c1_g2_w8", "flash_decoding_reduce_bf16_ext"]
    # 8 waves only where the keys set P and 4-wave blocks would overflow the
    # CUs: 2048 keys (32 partitions x 4 KV heads) and batch 8 (P set by the
    # CU count) keep 4 waves
    short = pa.Kernels.FlashAttention(q, T([1, 4, 2048, 256]), T([1, 4, 2048, 256]), out=o, scale=1 / 16, batch=1,
                                      query_heads=8, kv_heads=4, query_len=1, key_len=2048, head_dim=256)
    assert short.function_names[0] == "flash_decoding_partial_bf16_l32_c1_g2"
    k8 = T([8, 4, 8192, 256], "f16")
    wide = pa.Kernels.FlashAttention(T([8, 8, 1, 256], "f16"), k8, k8, out=T([8, 8, 1, 256], "f16"), scale=1 / 16,
                                     batch=8, query_heads=8, kv_heads=4, query_len=1, key_len=8192, head_dim=256)
    assert wide.function_names[0] == "flash_decoding_partial_f16_l32_c1_g2"
    f = pa.Kernels.FlashAttention(T([1, 4, 1, 64], "f32"), T([1, 1, 129, 64], "f32"), T([1, 1, 129, 64], "f32"),
                                  T([1, 4, 1, 64], "f32"), scale=0.125)
    assert f.function_names[0] == "flash_decoding_partial_f32_l16_c1_g4"
    g = pa.Kernels.FlashAttention(T([1, 2, 1, 80]), T([1, 1, 9, 80]), T([1, 1, 9, 80]), T([1, 2, 1, 80], "f32"),
                                  scale=0.1)
    assert g.function_names == ["flash_decoding_partial_bf16_ext", "flash_decoding_reduce_f32_ext"]


def test_flash_attention_validation_codes():
    E = pa.PopcornError
    cases = [
        (lambda: pa.Kernels.FlashAttention(T([1, 3, 1, 64]), T([1, 2, 9, 64]), T([1, 2, 9, 64]), T([1, 3, 1, 64]),
                                           scale=1.0), E.TENSOR_SHAPE_MISMATCH),  # 3 % 2 != 0
        (lambda: pa.Kernels.FlashAttention(T([1, 2, 1, 520]), T([1, 2, 9, 520]), T([1, 2, 9, 520]),
                                           T([1, 2, 1, 520]), scale=1.0), E.TENSOR_SHAPE_MISMATCH),  # Hd > 512
        (lambda: pa.Kernels.FlashAttention(T([2, 1, 64]), T([1, 2, 9, 64]), T([1, 2, 9, 64]), T([1, 2, 1, 64]),
                                           scale=1.0), E.TENSOR_INVALID_RANK),
        (lambda: pa.Kernels.FlashAttention(T([1, 2, 1, 64]), T([1, 2, 9, 64]), T([1, 2, 9, 64]), T([1, 2, 2, 64]),
                                           scale=1.0), E.TENSOR_SHAPE_MISMATCH),
        (lambda: pa.Kernels.FlashAttention(T([1, 2, 1, 64], "i32"), T([1, 2, 9, 64], "i32"),
                                           T([1, 2, 9, 64], "i32"), T([1, 2, 1, 64]), scale=1.0),
         E.UNSUPPORTED_DATA_TYPE_COMBINATION),
        # dims init reading past a too-small K tensor is refused
        (lambda: pa.Kernels.FlashAttention(T([1, 2, 1, 64]), T([1, 2, 9, 64]), T([1, 2, 9, 64]), T([1, 2, 1, 64]),
                                           scale=1.0, batch=1, query_heads=2, kv_heads=2, query_len=1, key_len=10,
                                           head_dim=64), E.TENSOR_SHAPE_MISMATCH),
    ]
    for make, code in cases:
        with pytest.raises(pa.PopcornError) as e:
            make()
        assert e.value.code == code, e.value


def test_matmul_routing_and_validation():
    x = T([1, 2304])
    # 4 rows per unit for long outputs (the LM head), 1 otherwise
    assert pa.Kernels.Matmul(x, T([32768, 2304]), T([1, 32768]), True).describe() == "matvec_nk_stream_bf16_bf16_bf16_r4"
    assert pa.Kernels.Matmul(x, T([9216, 2304]), T([1, 9216]), True).describe() == "matvec_nk_stream_bf16_bf16_bf16_r1"
    assert pa.Kernels.Matmul(T([1, 9216]), T([2304, 9216]), T([1, 2304]), True).describe() == \
        "matvec_nk_stream_bf16_bf16_bf16_r1"
    assert pa.Kernels.Matmul(x, T([2304, 300]), T([1, 300]), False).describe() == "matvec_bf16_bf16_bf16"
    assert pa.Kernels.Matmul(T([4, 8], "f32"), T([8, 4], "f32"), T([4, 4], "f32")).describe() == "matmul_mfma_f32_f32_f32"
    assert pa.Kernels.Matmul(T([4, 8], "f32"), T([8, 3], "f32"), T([4, 3], "f32")).describe() == "matmul_tiled"  # N % 4
    assert pa.Kernels.Matmul(T([64, 256], "f32"), T([300, 256]), T([64, 300], "f32"), True).describe() == \
        "matmul_mfma_f32_bf16_f32_tb"
    assert pa.Kernels.Matmul(T([64, 256]), T([256, 300], "f32"), T([64, 300], "f32"), False).describe() == \
        "matmul_mfma_bf16_f32_f32"
    # a 16-bit [K, N] B: transposed into scratch, then the matrix-core route
    assert pa.Kernels.Matmul(T([2048, 3072]), T([3072, 3072]), T([2048, 3072]), False).describe().startswith(
        "transpose2d_b16,matmul_mfma_bf16_bf16_bf16_")
    assert pa.Kernels.Matmul(T([8, 2304]), T([2304, 9216]), T([8, 9216], "f32"), False).describe() == \
        "transpose2d_b16,matmul_skinny_bf16_bf16_f32_m16_lds"
    assert pa.Kernels.Matmul(T([8, 2300]), T([2300, 64]), T([8, 64]), False).describe() == "matmul_tiled_bf16_bf16_bf16"
    with pytest.raises(pa.PopcornError) as e:  # Matmul.swift:85-87
        pa.Kernels.Matmul(x, T([9216, 2300]), T([1, 9216]), True)
    assert e.value.code == pa.PopcornError.TENSOR_SHAPE_MISMATCH
    with pytest.raises(pa.PopcornError) as e:
        pa.Kernels.Matmul(T([2304]), T([9216, 2304]), T([1, 9216]), True)
    assert e.value.code == pa.PopcornError.TENSOR_INVALID_RANK
    with pytest.raises(pa.PopcornError) as e:
        pa.Kernels.Matmul(T([1, 8], "i32"), T([8, 8], "i32"), T([1, 8], "i32"), True)
    assert e.value.code == pa.PopcornError.UNSUPPORTED_DATA_TYPE_COMBINATION


def test_rmsnorm_kv_elementwise_validation():
    E = pa.PopcornError
    with pytest.raises(E) as e:
        pa.Kernels.RMSNorm(T([2, 8]), None, T([2, 8]), axis=0, eps=1e-6)
    assert e.value.code == E.TENSOR_INVALID_AXIS
    with pytest.raises(E) as e:
        pa.Kernels.RMSNorm(T([2, 8]), T([8], "bf16"), T([2, 8]), eps=1e-6)  # weight must be f32
    assert e.value.code == E.UNSUPPORTED_DATA_TYPE_COMBINATION
    assert pa.Kernels.RMSNorm(T([2, 8]), T([8], "f32"), T([2, 8]), eps=1e-6).describe() == "rmsnorm_bf16"
    with pytest.raises(E) as e:
        pa.Kernels.KVCacheWrite(T([1, 4, 1, 256]), T([1, 4, 10, 256]), offset=10)
    assert e.value.code == E.TENSOR_SHAPE_MISMATCH
    assert pa.Kernels.KVCacheWrite(T([1, 4, 1, 256], "f32"), T([1, 4, 10, 256]), offset=9).describe() == \
        "kv_cache_write_f32_to_bf16"
    with pytest.raises(E) as e:
        pa.Kernels.Mul(T([4]), T([5]), T([4]))
    assert e.value.code == E.TENSOR_SHAPE_MISMATCH
    assert pa.Kernels.GeluTanh(T([7], "f16"), T([7], "f16")).describe() == "gelu_tanh_f16"


def test_rope_transpose_validation_and_routing():
    # RopeBuildCosSin.swift:37-48, RopeApply.swift:18-30 and :47-58, Transpose12.swift:15-20 and :27-35
    E = pa.PopcornError
    pos, inv = T([6], "i32"), T([64], "f32")
    cs = [T([6, 64], "f32", FAKE + 2 ** 20), T([6, 64], "f32", FAKE + 2 ** 21)]
    assert pa.Kernels.RopeBuildCosSin(pos, inv, *cs).describe() == "rope_build_cos_sin"
    with pytest.raises(E) as e:
        pa.Kernels.RopeBuildCosSin(T([5], "i32"), inv, *cs)
    assert e.value.code == E.TENSOR_SHAPE_MISMATCH and "positions count must equal seqLen 6" in str(e.value)
    with pytest.raises(E) as e:
        pa.Kernels.RopeBuildCosSin(pos, inv, T([6, 64], "f32"), T([6, 32], "f32"))
    assert e.value.code == E.TENSOR_SHAPE_MISMATCH
    with pytest.raises(E) as e:
        pa.Kernels.RopeBuildCosSin(pos, inv, T([6, 64, 1], "f32"), T([6, 64, 1], "f32"))
    assert e.value.code == E.TENSOR_INVALID_RANK
    x = T([1, 6, 8, 128])
    for xt, tt, name in (("f32", "f32", "rope_apply"), ("bf16", "bf16", "rope_apply_bf16"),
                         ("bf16", "f32", "rope_apply_f32_tables_bf16")):
        k = pa.Kernels.RopeApply(T([1, 6, 8, 128], xt), T([6, 64], tt), T([6, 64], tt),
                                 T([1, 6, 8, 128], xt, FAKE + 2 ** 24))
        assert k.describe() == name
    with pytest.raises(E) as e:
        pa.Kernels.RopeApply(T([1, 6, 8, 128], "f16"), T([6, 64], "f16"), T([6, 64], "f16"), T([1, 6, 8, 128], "f16"))
    assert e.value.code == E.UNSUPPORTED_DATA_TYPE_COMBINATION
    with pytest.raises(E) as e:
        pa.Kernels.RopeApply(x, T([6, 32], "f32"), T([6, 32], "f32"), T([1, 6, 8, 128]))
    assert e.value.code == E.TENSOR_SHAPE_MISMATCH and "tables must have shape [6, 64]" in str(e.value)
    with pytest.raises(E) as e:
        pa.Kernels.RopeApply(T([1, 6, 8, 7]), T([6, 3]), T([6, 3]), T([1, 6, 8, 7]), batch=1, seq_len=6,
                             head_count=8, head_dim=7)
    assert e.value.code == E.TENSOR_SHAPE_MISMATCH and "must be even" in str(e.value)
    for dt, name in (("f32", "transpose12"), ("f16", "transpose12_f16"), ("bf16", "transpose12_bf16")):
        assert pa.Kernels.Transpose12(T([1, 6, 8, 128], dt), T([1, 8, 6, 128], dt)).describe() == name
    with pytest.raises(E) as e:
        pa.Kernels.Transpose12(T([1, 6, 8, 128]), T([1, 6, 8, 128]))
    assert e.value.code == E.TENSOR_SHAPE_MISMATCH and "must be [1, 8, 6, 128]" in str(e.value)
    with pytest.raises(E) as e:
        pa.Kernels.Transpose12(T([1, 6, 8, 128], "i32"), T([1, 8, 6, 128], "i32"))
    assert e.value.code == E.UNSUPPORTED_DATA_TYPE_COMBINATION


def _q4(out, inn, scale_dt="bf16", bias=True, packed_dt="u32", bias_shape=None, ptr=FAKE + 2 ** 33, rank2=True):
    packed = T([out, inn // 8], packed_dt, ptr)
    scales = T([out, inn // 64], scale_dt, ptr + 2 ** 30)
    biases = T(bias_shape or [out, inn // 64], scale_dt, ptr + 2 ** 31) if bias else None
    return pa.AffineQuantizedTensor(packed, scales, biases, [out, inn] if rank2 else [inn])


def test_quantized_validation_and_routing():
    # AffineQuantizedTensor.swift:29-48, Matmul.swift:99-130 / :279-332, EmbeddingGather.swift:45-88
    E = pa.PopcornError
    for kw, code in ((dict(packed_dt="f32"), E.UNSUPPORTED_DATA_TYPE_COMBINATION),
                     (dict(bias_shape=[10, 3]), E.TENSOR_SHAPE_MISMATCH),
                     (dict(rank2=False), E.TENSOR_INVALID_RANK)):
        with pytest.raises(E) as e:
            _q4(9216, 2304, **kw)
        assert e.value.code == code
    w = _q4(9216, 2304)
    out = T([1, 9216], "bf16", FAKE + 2 ** 20)
    assert pa.Kernels.Matmul(T([1, 2304]), w, out).describe() == "aq_qmv_fast_bf16_bf16_bf16_b4_g64_l12_j2"
    assert pa.Kernels.Matmul(T([4, 2304]), w, T([4, 9216], "f32")).describe() == "aq_matvec_simd4_bf16_bf16_f32_b4_g64_l12_j2"
    # bf16 rows reading >= 2^27 weight bytes in all (and m >= 16): the
    # matrix-core GEMM, group sums and pair-ordered x first; few tiles split
    # the K groups over blocks, summed by the split-K reduction
    assert pa.Kernels.Matmul(T([15, 2304]), w, T([15, 9216], "f32")).describe() == "aq_matvec_simd4_bf16_bf16_f32_b4_g64_l12_j2"
    assert pa.Kernels.Matmul(T([16, 2304]), w, T([16, 9216], "f32")).describe() == \
        "aq_gemm_prep_bf16,aq_gemm_mfma_bf16_bf16_splitk_b4_g64,matmul_splitk_reduce_f32"
    assert pa.Kernels.Matmul(T([16, 1024]), _q4(16000, 1024), T([16, 16000], "f32")).describe().startswith("aq_matvec")
    assert pa.Kernels.Matmul(T([2048, 2304]), w, T([2048, 9216])).describe() == \
        "aq_gemm_prep_bf16,aq_gemm_mfma_bf16_bf16_bf16_b4_g64"
    assert pa.Kernels.Matmul(T([64, 2304], "f32"), w, T([64, 9216], "f32")).describe().startswith("aq_matvec_simd4_f32")
    down = _q4(2304, 9216)
    assert pa.Kernels.Matmul(T([16, 9216]), down, T([16, 2304], "f32")).describe() == \
        "aq_gemm_prep_bf16,aq_gemm_mfma_bf16_bf16_splitk_b4_g64,matmul_splitk_reduce_f32"
    assert pa.Kernels.Matmul(T([1, 9216]), down, T([1, 2304])).describe() == "aq_qmv_fast_bf16_bf16_bf16_b4_g64_l16_j8"
    # unaligned activations or f32 x past 4096 take the any-shape kernel
    assert pa.Kernels.Matmul(T([1, 2304], ptr=FAKE + 2), w, out).describe() == "aq_matvec_simd4_bf16_bf16_bf16_b4_g64"
    assert pa.Kernels.Matmul(T([1, 9216], "f32"), down, T([1, 2304], "f32")).describe() == \
        "aq_matvec_simd4_f32_bf16_f32_b4_g64"
    with pytest.raises(E) as e:
        pa.Kernels.Matmul(T([1, 2300]), w, out)
    assert e.value.code == E.TENSOR_SHAPE_MISMATCH and "b.inFeatures=2304" in str(e.value)
    with pytest.raises(E) as e:
        pa.Kernels.Matmul(T([1, 2304], "f16"), w, T([1, 9216], "f16"))
    assert e.value.code == E.UNSUPPORTED_DATA_TYPE_COMBINATION
    with pytest.raises(E) as e:
        pa.Kernels.Matmul(T([1, 2304]), w, T([1, 9215]))
    assert e.value.code == E.TENSOR_SHAPE_MISMATCH
    with pytest.raises(E) as e:
        pa.Kernels.Matmul(T([1, 96]), _q4(8, 96 + 32), T([1, 8]))
    assert e.value.code == E.TENSOR_SHAPE_MISMATCH
    emb = _q4(256000, 2304)
    ids = T([3], "i32")
    assert pa.Kernels.EmbeddingGather(ids, emb, T([3, 2304])).describe() == "aq_embedding_gather_bf16_bf16_b4_g64_ext"
    with pytest.raises(E) as e:
        pa.Kernels.EmbeddingGather(T([3], "i64"), emb, T([3, 2304]))
    assert e.value.code == E.UNSUPPORTED_DATA_TYPE_COMBINATION
    with pytest.raises(E) as e:
        pa.Kernels.EmbeddingGather(ids, emb, T([3, 2300]))
    assert e.value.code == E.TENSOR_SHAPE_MISMATCH


def test_gated_mlp_validation_and_routing():
    E = pa.PopcornError
    k = pa.Kernels.GatedMLP(T([2304]), T([2304], "f32"), T([9216, 2304]), T([9216, 2304]), T([2304, 9216]),
                            T([2304]), eps=1e-6)
    assert k.function_names == ["gated_mlp_gate_up_bf16_r1", "matvec_nk_stream_bf16_bf16_bf16_r1"]
    r = pa.Kernels.GatedMLPResidual(T([2304]), T([2304]), T([2304], "f32"), T([2304], ptr=FAKE + 4096), T([2304], "f32"),
                                    T([9216, 2304]), T([9216, 2304]), T([2304, 9216]), T([2304]), eps=1e-6)
    assert r.function_names == ["gated_mlp_gate_up_bf16_r1_res", "matvec_nk_stream_bf16_bf16_bf16_r1"]
    with pytest.raises(E) as e:
        pa.Kernels.GatedMLP(T([2304]), None, T([9216, 2304]), T([9216, 2300]), T([2304, 9216]), T([2304]), eps=1e-6)
    assert e.value.code == E.TENSOR_SHAPE_MISMATCH
    with pytest.raises(E) as e:
        pa.Kernels.GatedMLP(T([2304]), None, T([9216, 2304]), T([9216, 2304], "f16"), T([2304, 9216]), T([2304]),
                            eps=1e-6)
    assert e.value.code == E.UNSUPPORTED_DATA_TYPE_COMBINATION


def test_custom_kernel_rejects_empty_access():
    # Tensor.swift:208: a binding's access must not be empty
    with pytest.raises(pa.PopcornError) as e:
        pa.Kernels.Custom("add", [T([4], "f32")], [0], [], (1, 1, 1), (64, 1, 1))
    assert e.value.code == pa.PopcornError.INVALID_ARGUMENT


def test_no_gpu_paths_fail_loudly_here():
    if pa.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(pa.PopcornError):
        pa.KernelLibrary()


def test_decode_matvec_routing():
    # the glue is compiled in: _f<bit0 residual | bit1 pre-norm>; the KV
    # scatter is a runtime flag; 4 rows per unit for long outputs
    x, w = T([2304]), T([4096, 2304])
    norm = T([2304], "f32")
    caches = dict(k_cache=T([4, 4352, 256], ptr=FAKE + 2 ** 30), v_cache=T([4, 4352, 256], ptr=FAKE + 2 ** 31),
                  position=T([1], "i32"), q_rows=2048)
    assert pa.Kernels.DecodeMatvec(x, T([2048, 2304]), T([2048])).function_names == ["decode_matvec_bf16_bf16_r1_f0"]
    assert pa.Kernels.DecodeMatvec(x, w, T([2048]), w_pre=norm, **caches).function_names == \
        ["decode_matvec_bf16_bf16_r1_f2"]
    res = dict(delta=T([2304]), w_post=norm, x_out=T([2304], ptr=FAKE + 2 ** 20))
    assert pa.Kernels.DecodeMatvec(x, w, T([2048]), w_pre=norm, **res, **caches).function_names == \
        ["decode_matvec_bf16_bf16_r1_f3"]
    assert pa.Kernels.DecodeMatvec(x, T([256000, 2304]), T([256000], "f32"), w_pre=norm, **res).function_names == \
        ["decode_matvec_bf16_f32_r4_f3"]
    E = pa.PopcornError
    with pytest.raises(E) as e:  # rows must be q_rows + K rows + V rows
        pa.Kernels.DecodeMatvec(x, T([4000, 2304]), T([2048]), **caches)
    assert e.value.code == E.TENSOR_SHAPE_MISMATCH
    with pytest.raises(E) as e:  # the residual output may not alias x
        pa.Kernels.DecodeMatvec(x, w, T([4096]), delta=T([2304]), w_post=norm, x_out=x)
    assert e.value.code == E.INVALID_ARGUMENT


def test_prefill_routes_to_tiled():
    # FlashAttention.swift:109-113 with the MFMA kernel in the MPP role
    assert pa.Kernels.route(2048, 256, "f16") == "tiled"
    assert pa.Kernels.route(32, 64, "bf16") == "tiled"
    assert pa.Kernels.route(31, 64, "bf16") == "plain"
    assert pa.Kernels.route(2048, 80, "f16") == "tiled"
    assert pa.Kernels.route(2048, 512, "bf16") == "tiled"
    assert pa.Kernels.route(2048, 36, "f16") == "plain"     # rows not in 16-byte chunks
    assert pa.Kernels.route(2048, 520, "f16") == "plain"
    assert pa.Kernels.route(2048, 256, "f32") == "tiled"     # v_mfma_f32_16x16x4_f32
    assert pa.Kernels.route(2048, 36, "f32") == "tiled"      # f32 rows in 16-byte chunks
    assert pa.Kernels.route(2048, 34, "f32") == "plain"
    assert pa.Kernels.route(31, 256, "f32") == "plain"
    assert pa.Kernels.route(1, 256, "f16") == "decoding"
    q = T([1, 16, 2048, 256], "f16")
    k = pa.Kernels.FlashAttention(q, q, q, out=T([1, 16, 2048, 256], "f16", ptr=FAKE + 2 ** 32), scale=1 / 16)
    assert k.function_names == ["flash_attention_tiled16_f16_f16_d256"]
    for hd, hdp in ((64, 64), (80, 128), (256, 256), (320, 512)):
        qf = T([1, 4, 256, hd], "f32")
        kf = pa.Kernels.FlashAttention(qf, qf, qf, out=T([1, 4, 256, hd], "f32", ptr=FAKE + 2 ** 32), scale=0.1)
        assert kf.function_names == [f"flash_attention_tiled16_f32_f32_d{hdp}"]


# Reference kernels outside the decode hot path (the reference's own unfused
# attention, LayerNorm/GroupNorm, softmax, slicing, broadcast add, soft-cap):
# not built here.
OUT_OF_SCOPE = ("attention_output", "attention_scores", "broadcast_add", "groupnorm", "layernorm", "logit_softcap",
                "row_slice2d", "slice2d", "softmax")


def test_reference_named_kernels_take_the_reference_parameter_lists():
    # tests/golden/reference_kernel_abi.json lists every kernel the reference
    # instantiates with its parameter list (device pointers, then the byte
    # size of each constants block), written from the Metal sources by
    # tests/golden/make_reference_abi.py. Every one on the hot path is
    # exported under the same name and takes exactly that list, read back
    # from this build's code objects; a raw launch packed like the
    # reference's therefore matches the kernel.
    ref = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_kernel_abi.json")))
    assert ref["kv_cache_write"] == {"buffers": 2, "constants": [24], "source": "Sources/Popcorn/Kernels/KVCacheWrite.metal:7"}
    assert ref["flash_decoding_partial_bf16"]["buffers"] == 6 and ref["flash_decoding_partial_bf16"]["constants"] == [36]
    files = sorted(glob.glob(os.path.join(pa.KERNEL_DIR, "*.hsaco")))
    assert files
    required = [n for n in ref if not n.startswith(OUT_OF_SCOPE)]
    assert len(required) == 58
    for name in required:
        got = None
        for f in files:
            try:
                got = pa.code_object_layout(f, name)
                break
            except pa.PopcornError as e:
                assert e.code == -1006, e
        assert got is not None, f"{name} is not exported"
        assert (got["buffers"], got["constants"]) == (ref[name]["buffers"], ref[name]["constants"]), (name, got, ref[name])


def test_extended_kernels_have_names_of_their_own():
    # the forms with this build's extra parameters (device position, KV row
    # stride, bounds on table ids) carry an _ext suffix and their own
    # constants blocks
    f = os.path.join(pa.KERNEL_DIR, "kv_cache_write.hsaco")
    assert pa.code_object_layout(f, "kv_cache_write_bf16_ext")["buffers"] == 3
    assert pa.code_object_layout(f, "kv_cache_write_bf16_ext")["constants"] == [28]
    fd = os.path.join(pa.KERNEL_DIR, "flash_decoding.hsaco")
    assert pa.code_object_layout(fd, "flash_decoding_partial_bf16_ext")["constants"] == [48]
    assert pa.code_object_layout(fd, "flash_decoding_reduce_bf16_ext")["constants"] == [20]
    with pytest.raises(pa.PopcornError) as e:
        pa.code_object_layout(fd, "no_such_kernel")
    assert e.value.code == -1006
    with pytest.raises(pa.PopcornError) as e:
        pa.code_object_layout(os.path.join(ROOT, "README.md"), "kv_cache_write")
    assert e.value.code == -1100
