"""ctypes declarations of include/popcorn_hip.h (the C ABI of libpopcorn_amd.so).

The library is built in-tree by ``__graft_entry__.build()`` (or ``make -C
popcorn_amd/csrc``). Importing this module without it raises: there is no
fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libpopcorn_amd.so")
KERNEL_DIR = os.path.join(LIB_DIR, "kernels")

MAX_RANK = 8

# dtype tags (Tensor.DataType order, Tensor.swift:136-148)
DTYPES = {"u8": 0, "u16": 1, "u32": 2, "u64": 3, "i8": 4, "i16": 5, "i32": 6, "i64": 7,
          "f32": 8, "f16": 9, "bf16": 10}
DTYPE_NAMES = {v: k for k, v in DTYPES.items()}


class TensorDesc(C.Structure):
    _fields_ = [("data", C.c_void_p), ("dtype", C.c_int32), ("rank", C.c_int32),
                ("shape", C.c_int64 * MAX_RANK)]


class AttentionMaskDesc(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("window", C.c_int32)]


class AffineQuantizedDesc(C.Structure):
    _fields_ = [("packed_values", TensorDesc), ("scales", TensorDesc), ("biases", TensorDesc),
                ("rank", C.c_int32), ("shape", C.c_int64 * MAX_RANK), ("bits", C.c_int32),
                ("group_size", C.c_int32)]


class SafetensorsInfo(C.Structure):
    _fields_ = [("name", C.c_char * 256), ("dtype_name", C.c_char * 16), ("dtype", C.c_int32), ("rank", C.c_int32),
                ("shape", C.c_int64 * MAX_RANK), ("offset", C.c_uint64), ("nbytes", C.c_uint64),
                ("index", C.c_int32)]


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("arch", C.c_char * 32), ("compute_units", C.c_int32),
                ("wave_size", C.c_int32), ("max_threads_per_block", C.c_int32),
                ("lds_bytes_per_block", C.c_int32), ("global_memory_bytes", C.c_int64),
                ("l2_bytes", C.c_int32), ("clock_khz", C.c_int32)]


class FunctionAttrs(C.Structure):
    _fields_ = [("max_threads_per_block", C.c_int32), ("wave_size", C.c_int32),
                ("static_lds_bytes", C.c_int32), ("num_vgprs", C.c_int32), ("num_sgprs", C.c_int32),
                ("private_bytes", C.c_int32)]


class KernelLayout(C.Structure):
    _fields_ = [("nbuffers", C.c_int32), ("nconstants", C.c_int32), ("constant_sizes", C.c_uint32 * 8),
                ("trailing_pointers", C.c_int32), ("max_threads_per_block", C.c_uint32)]


class EncoderStats(C.Structure):
    _fields_ = [("dispatches", C.c_int64), ("hazards", C.c_int64), ("scratch_borrows", C.c_int64)]


BORROW_FN = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p), C.POINTER(C.c_int32))
RELEASE_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_void_p)


class ScratchAllocatorDesc(C.Structure):
    _fields_ = [("context", C.c_void_p), ("borrow", BORROW_FN), ("release", RELEASE_FN)]


class DecoderConfig(C.Structure):
    _fields_ = [("layers", C.c_int32), ("hidden", C.c_int32), ("query_heads", C.c_int32),
                ("kv_heads", C.c_int32), ("head_dim", C.c_int32), ("ffn", C.c_int32), ("vocab", C.c_int32),
                ("max_seq", C.c_int32), ("eps", C.c_float), ("attn_scale", C.c_float),
                ("history_len", C.c_int32), ("graph_steps", C.c_int32), ("attention_block", C.c_int32),
                ("rope_theta", C.c_float), ("weight_bits", C.c_int32)]


_T = C.POINTER(TensorDesc)


class DecodeMatvecArgs(C.Structure):
    _fields_ = [(n, _T) for n in ("x", "delta", "w_post", "x_out", "w_pre", "weight", "out", "k_cache", "v_cache",
                                  "position")] + [("q_rows", C.c_int64), ("eps", C.c_float),
                                                  ("qweight", C.POINTER(AffineQuantizedDesc))]


class DecodeAttentionArgs(C.Structure):
    _fields_ = [(n, _T) for n in ("qkv", "k_cache", "v_cache", "out", "position", "q_norm", "k_norm",
                                  "inv_freq")] + [("v_norm", C.c_int32), ("query_heads", C.c_int32),
                                                  ("kv_heads", C.c_int32), ("eps", C.c_float),
                                                  ("scale", C.c_float), ("rope_scaling", C.c_float),
                                                  ("mask", AttentionMaskDesc)]


_K = C.POINTER(C.c_void_p)
_st = C.c_int32

# name -> (restype, argtypes); every function returning popcorn_status_t is checked
PROTOTYPES = {
    "popcorn_last_error_message": (C.c_char_p, []),
    "popcorn_status_from_hip_error": (_st, [C.c_int]),
    "popcorn_dtype_stride": (C.c_int32, [C.c_int32]),
    "popcorn_device_count": (_st, [C.POINTER(C.c_int32)]),
    "popcorn_set_device": (_st, [C.c_int32]),
    "popcorn_device_info": (_st, [C.c_int32, C.POINTER(DeviceInfo)]),
    "popcorn_device_synchronize": (_st, []),
    "popcorn_malloc": (_st, [C.c_size_t, C.POINTER(C.c_void_p)]),
    "popcorn_free": (_st, [C.c_void_p]),
    "popcorn_malloc_uncached": (_st, [C.c_size_t, C.POINTER(C.c_void_p)]),
    "popcorn_free_uncached": (_st, [C.c_void_p]),
    "popcorn_memcpy_h2d": (_st, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "popcorn_memcpy_d2h": (_st, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "popcorn_memcpy_d2d": (_st, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "popcorn_memset": (_st, [C.c_void_p, C.c_int32, C.c_size_t, C.c_void_p]),
    "popcorn_stream_create": (_st, [C.POINTER(C.c_void_p)]),
    "popcorn_stream_destroy": (_st, [C.c_void_p]),
    "popcorn_stream_synchronize": (_st, [C.c_void_p]),
    "popcorn_attention_pair_flags": (_st, [C.c_void_p, C.POINTER(C.c_void_p), C.POINTER(C.c_int32)]),
    "popcorn_event_create": (_st, [C.POINTER(C.c_void_p)]),
    "popcorn_event_destroy": (_st, [C.c_void_p]),
    "popcorn_event_record": (_st, [C.c_void_p, C.c_void_p]),
    "popcorn_event_wait": (_st, [C.c_void_p, C.c_void_p]),
    "popcorn_event_synchronize": (_st, [C.c_void_p]),
    "popcorn_event_elapsed_ms": (_st, [C.c_void_p, C.c_void_p, C.POINTER(C.c_float)]),
    "popcorn_library_load": (_st, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "popcorn_library_destroy": (_st, [C.c_void_p]),
    "popcorn_library_function": (_st, [C.c_void_p, C.c_char_p, C.POINTER(C.c_void_p)]),
    "popcorn_function_attributes": (_st, [C.c_void_p, C.POINTER(FunctionAttrs)]),
    "popcorn_function_layout": (_st, [C.c_void_p, C.POINTER(KernelLayout)]),
    "popcorn_code_object_layout": (_st, [C.c_char_p, C.c_char_p, C.POINTER(KernelLayout)]),
    "popcorn_library_cached_function_count": (C.c_int32, [C.c_void_p]),
    "popcorn_launch": (_st, [C.c_void_p, C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                             C.POINTER(C.c_void_p), C.c_int32, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t),
                             C.c_int32, C.c_size_t]),
    "popcorn_scratch_pool_create": (_st, [C.POINTER(C.c_void_p)]),
    "popcorn_scratch_pool_destroy": (_st, [C.c_void_p]),
    "popcorn_scratch_pool_allocator": (_st, [C.c_void_p, C.POINTER(ScratchAllocatorDesc)]),
    "popcorn_scratch_pool_bytes": (C.c_size_t, [C.c_void_p]),
    "popcorn_scratch_spec_byte_count": (C.c_size_t, [C.POINTER(C.c_int64), C.c_int32, C.c_int32]),
    "popcorn_encoder_create": (_st, [C.c_void_p, C.c_void_p, C.POINTER(ScratchAllocatorDesc), C.POINTER(C.c_void_p)]),
    "popcorn_encoder_destroy": (_st, [C.c_void_p]),
    "popcorn_encoder_encode": (_st, [C.c_void_p, C.c_void_p]),
    "popcorn_encoder_encode_all": (_st, [C.c_void_p, C.POINTER(C.c_void_p), C.c_int32]),
    "popcorn_encoder_barrier": (_st, [C.c_void_p]),
    "popcorn_encoder_stats": (_st, [C.c_void_p, C.POINTER(EncoderStats)]),
    "popcorn_flash_attention_route": (C.c_int32, [C.c_int64, C.c_int64, C.c_int32]),
    "popcorn_kernel_flash_attention": (_st, [_T, _T, _T, _T, C.c_float, AttentionMaskDesc, _K]),
    "popcorn_kernel_flash_attention_dims": (_st, [_T, _T, _T, _T, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
                                                  C.c_int64, C.c_int64, C.c_float, AttentionMaskDesc, C.c_int64,
                                                  _T, _K]),
    "popcorn_flash_decoding_no_alloc": (_st, [C.c_void_p, C.c_void_p, _T, _T, _T, _T, C.c_int64, C.c_int64,
                                              C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_float,
                                              AttentionMaskDesc, C.c_int64, _T]),
    "popcorn_kernel_matmul": (_st, [_T, _T, _T, C.c_int32, _K]),
    "popcorn_kernel_matmul_dims": (_st, [_T, _T, _T, C.c_int64, C.c_int64, C.c_int64, C.c_int32, _K]),
    "popcorn_kernel_rmsnorm": (_st, [_T, _T, _T, C.c_int32, C.c_float, C.c_int32, _K]),
    "popcorn_kernel_rmsnorm_dims": (_st, [_T, _T, _T, C.c_int64, C.c_int64, C.c_float, C.c_int32, _K]),
    "popcorn_kernel_kv_cache_write": (_st, [_T, _T, C.c_int64, _K]),
    "popcorn_kernel_kv_cache_write_dims": (_st, [_T, _T, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
                                                 C.c_int64, _T, _K]),
    "popcorn_kernel_gelu_tanh": (_st, [_T, _T, _K]),
    "popcorn_kernel_mul": (_st, [_T, _T, _T, _K]),
    "popcorn_kernel_add": (_st, [_T, _T, _T, _K]),
    "popcorn_kernel_scalar_mul": (_st, [_T, C.c_float, _T, _K]),
    "popcorn_kernel_rope_build_cos_sin": (_st, [_T, _T, _T, _T, C.c_float, _K]),
    "popcorn_kernel_rope_build_cos_sin_dims": (_st, [_T, _T, _T, _T, C.c_int64, C.c_int64, C.c_float, _K]),
    "popcorn_kernel_rope_apply": (_st, [_T, _T, _T, _T, _K]),
    "popcorn_kernel_rope_apply_dims": (_st, [_T, _T, _T, _T, C.c_int64, C.c_int64, C.c_int64, C.c_int64, _K]),
    "popcorn_kernel_transpose12": (_st, [_T, _T, _K]),
    "popcorn_kernel_transpose12_dims": (_st, [_T, _T, C.c_int64, C.c_int64, C.c_int64, C.c_int64, _K]),
    "popcorn_kernel_gated_mlp": (_st, [_T, _T, _T, _T, _T, _T, C.c_float, C.c_int32, _T, _K]),
    "popcorn_kernel_gated_mlp_residual": (_st, [_T, _T, _T, _T, _T, _T, _T, _T, _T, C.c_float, C.c_int32, _T, _K]),
    "popcorn_kernel_decode_matvec": (_st, [C.POINTER(DecodeMatvecArgs), _K]),
    "popcorn_kernel_gated_mlp_residual_quantized": (_st, [_T, _T, _T, _T, _T, C.POINTER(AffineQuantizedDesc),
                                                          C.POINTER(AffineQuantizedDesc),
                                                          C.POINTER(AffineQuantizedDesc), _T, C.c_float, _T, _K]),
    "popcorn_kernel_decode_attention": (_st, [C.POINTER(DecodeAttentionArgs), _K]),
    "popcorn_kernel_embedding_gather": (_st, [_T, _T, _T, _K]),
    "popcorn_affine_quantized_validate": (_st, [C.POINTER(AffineQuantizedDesc)]),
    "popcorn_kernel_matmul_quantized": (_st, [_T, C.POINTER(AffineQuantizedDesc), _T, _K]),
    "popcorn_kernel_embedding_gather_quantized": (_st, [_T, C.POINTER(AffineQuantizedDesc), _T, _K]),
    "popcorn_kernel_argmax": (_st, [_T, _T, _K]),
    "popcorn_kernel_custom": (_st, [C.c_char_p, _T, C.POINTER(C.c_uint8), C.c_int32, C.POINTER(C.c_void_p),
                                    C.POINTER(C.c_size_t), C.c_int32, C.POINTER(C.c_uint32),
                                    C.POINTER(C.c_uint32), _K]),
    "popcorn_kernel_destroy": (_st, [C.c_void_p]),
    "popcorn_kernel_describe": (_st, [C.c_void_p, C.c_char_p, C.c_size_t]),
    "popcorn_fill_normal": (_st, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_uint64, C.c_uint64,
                                  C.c_float, C.c_float]),
    # include/popcorn_safetensors.h
    "popcorn_safetensors_open": (_st, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "popcorn_safetensors_close": (_st, [C.c_void_p]),
    "popcorn_safetensors_count": (C.c_int32, [C.c_void_p]),
    "popcorn_safetensors_info": (_st, [C.c_void_p, C.c_int32, C.POINTER(SafetensorsInfo)]),
    "popcorn_safetensors_find": (_st, [C.c_void_p, C.c_char_p, C.POINTER(SafetensorsInfo)]),
    "popcorn_safetensors_metadata": (_st, [C.c_void_p, C.c_char_p, C.c_char_p, C.c_size_t]),
    "popcorn_safetensors_read": (_st, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_size_t]),
    "popcorn_safetensors_upload": (_st, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    # include/popcorn_decoder.h
    "popcorn_decoder_create": (_st, [C.c_void_p, C.c_void_p, C.POINTER(DecoderConfig), C.POINTER(C.c_void_p)]),
    "popcorn_decoder_destroy": (_st, [C.c_void_p]),
    "popcorn_decoder_randomize": (_st, [C.c_void_p, C.c_uint64]),
    "popcorn_decoder_tensor": (_st, [C.c_void_p, C.c_char_p, C.c_int32, _T]),
    "popcorn_decoder_reset": (_st, [C.c_void_p, C.c_int32, C.c_int32]),
    "popcorn_decoder_step": (_st, [C.c_void_p, C.c_int32, C.c_int32]),
    "popcorn_decoder_read": (_st, [C.c_void_p, C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
    "popcorn_decoder_describe": (_st, [C.c_void_p, C.c_char_p, C.c_size_t, C.POINTER(C.c_int32)]),
    "popcorn_decoder_step_bytes": (C.c_int64, [C.c_void_p, C.c_int32]),
    "popcorn_decoder_time_kernel": (_st, [C.c_void_p, C.c_char_p, C.c_int32, C.POINTER(C.c_float),
                                          C.POINTER(C.c_int32)]),
    "popcorn_decoder_time_kernel_in_step": (_st, [C.c_void_p, C.c_char_p, C.c_int32, C.POINTER(C.c_float),
                                          C.POINTER(C.c_int32)]),
}

_lib = None


def load():
    """Loads libpopcorn_amd.so and declares every prototype; raises if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build the HIP extension first (python -c "
                "'import __graft_entry__ as g; g.build()' or make -C popcorn_amd/csrc)")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib
