"""Python mirror of the reference's Swift API over the C ABI.

Names, argument meaning and errors follow Sources/Popcorn (cited per class):
``Tensor``, ``Kernels.*``, ``KernelCommandEncoder`` (``encode`` takes one
kernel or several, the result-builder form), ``KernelLibrary``,
``ScratchPool`` (a ``KernelScratchAllocator``) and ``PopcornError``. Device
memory is plain HIP memory owned by ``DeviceBuffer``; host data moves through
numpy arrays (bf16 as uint16 bit patterns).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Iterable, Optional, Sequence

import numpy as np

from . import _capi
from ._capi import DTYPES, DTYPE_NAMES, MAX_RANK, TensorDesc, AttentionMaskDesc


# ---- errors (PopcornError.swift:23-42) --------------------------------------

class PopcornError(Exception):
    """Carries the reference's PopcornError.Code raw value in ``code``."""

    CONSTANT_ALLOCATION_FAILED = -1001
    TENSOR_ALLOCATION_FAILED = -1003
    KERNEL_FUNCTION_NOT_FOUND = -1006
    TENSOR_SHAPE_MISMATCH = -1007
    TENSOR_INVALID_RANK = -1008
    TENSOR_INVALID_AXIS = -1009
    UNSUPPORTED_DATA_TYPE_COMBINATION = -1010
    GPU_OUT_OF_MEMORY = -1013
    GPU_TIMEOUT = -1014
    GPU_PAGE_FAULT = -1015
    GPU_INVALID_RESOURCE = -1016
    GPU_DEVICE_REMOVED = -1017
    GPU_INTERNAL = -1019
    INVALID_ARGUMENT = -1100

    def __init__(self, code: int, message: str):
        super().__init__(f"PopcornError({code}): {message}")
        self.code = code
        self.message = message


def lib():
    return _capi.load()


def check(status: int) -> None:
    if status != 0:
        msg = lib().popcorn_last_error_message()
        raise PopcornError(int(status), msg.decode() if msg else "")


# ---- device ------------------------------------------------------------------

def device_count() -> int:
    n = C.c_int32(0)
    check(lib().popcorn_device_count(C.byref(n)))
    return n.value


def device_info(device: int = 0) -> dict:
    info = _capi.DeviceInfo()
    check(lib().popcorn_device_info(device, C.byref(info)))
    return {"name": info.name.decode(), "arch": info.arch.decode(), "compute_units": info.compute_units,
            "wave_size": info.wave_size, "max_threads_per_block": info.max_threads_per_block,
            "lds_bytes_per_block": info.lds_bytes_per_block, "global_memory_bytes": info.global_memory_bytes,
            "l2_bytes": info.l2_bytes, "clock_khz": info.clock_khz}


def synchronize() -> None:
    check(lib().popcorn_device_synchronize())


class Stream:
    """An in-order HIP stream (None = the default stream)."""

    def __init__(self):
        h = C.c_void_p()
        check(lib().popcorn_stream_create(C.byref(h)))
        self.handle = h.value

    def synchronize(self) -> None:
        check(lib().popcorn_stream_synchronize(self.handle))

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().popcorn_stream_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _stream_handle(stream) -> Optional[int]:
    return None if stream is None else stream.handle


class Event:
    def __init__(self):
        h = C.c_void_p()
        check(lib().popcorn_event_create(C.byref(h)))
        self.handle = h.value

    def record(self, stream: Optional[Stream] = None) -> None:
        check(lib().popcorn_event_record(self.handle, _stream_handle(stream)))

    def synchronize(self) -> None:
        check(lib().popcorn_event_synchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0)
        check(lib().popcorn_event_elapsed_ms(self.handle, end.handle, C.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                lib().popcorn_event_destroy(self.handle)
        except Exception:
            pass


class DeviceBuffer:
    """Owned device memory (the MTLBuffer a Tensor views)."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        check(lib().popcorn_malloc(max(int(nbytes), 1), C.byref(p)))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    def __del__(self):
        try:
            if self.ptr:
                lib().popcorn_free(self.ptr)
        except Exception:
            pass


class UncachedBuffer:
    """Uncached device memory (popcorn_malloc_uncached): every access goes to
    memory, past the per-XCD L2 caches. Given back to the library's pool,
    never to the driver."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        check(lib().popcorn_malloc_uncached(max(int(nbytes), 1), C.byref(p)))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    def __del__(self):
        try:
            if self.ptr:
                lib().popcorn_free_uncached(self.ptr)
        except Exception:
            pass


def attention_pair_flags(stream: Optional["Stream"] = None) -> "Tensor":
    """The ready flags of the tiled prefill attention's merged pairs on
    `stream` (u64: the abort word, then one flag per split tile)."""
    p, n = C.c_void_p(), C.c_int32()
    check(lib().popcorn_attention_pair_flags(_stream_handle(stream), C.byref(p), C.byref(n)))
    return Tensor(p.value, [n.value], "u64")


# ---- tensors (Tensor.swift) ----------------------------------------------------

_NP = {"f32": np.float32, "f16": np.float16, "bf16": np.uint16, "i32": np.int32, "u8": np.uint8,
       "u16": np.uint16, "u32": np.uint32, "u64": np.uint64, "i8": np.int8, "i16": np.int16, "i64": np.int64}


def stride(dtype: str) -> int:
    return int(lib().popcorn_dtype_stride(DTYPES[dtype]))


def _host_array(arr: np.ndarray, dtype: str) -> np.ndarray:
    """Host storage for `dtype`: uint16 bit patterns are reinterpreted for
    f16 (never value-converted); other inputs convert to the storage type."""
    arr = np.asarray(arr)
    if dtype == "f16" and arr.dtype == np.uint16:
        return np.ascontiguousarray(arr).view(np.float16)
    return np.ascontiguousarray(arr, dtype=_NP[dtype])


class Tensor:
    """Tensor{buffer, shape, dataType}: a view of device memory (Tensor.swift:5-22).

    ``ptr`` may be any device address; ``owner`` keeps its buffer alive.
    """

    def __init__(self, ptr: int, shape: Sequence[int], dtype: str = "f32", owner=None):
        if dtype not in DTYPES:
            raise ValueError(f"unknown dtype {dtype}")
        if len(shape) > MAX_RANK:
            raise ValueError("rank above 8")
        self.ptr = int(ptr) if ptr else 0
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        self.owner = owner

    # construction
    @classmethod
    def empty(cls, shape: Sequence[int], dtype: str = "f32") -> "Tensor":
        n = int(np.prod(shape)) if len(shape) else 1
        buf = DeviceBuffer(n * stride(dtype))
        return cls(buf.ptr, shape, dtype, owner=buf)

    @classmethod
    def empty_uncached(cls, shape: Sequence[int], dtype: str = "f32") -> "Tensor":
        n = int(np.prod(shape)) if len(shape) else 1
        buf = UncachedBuffer(n * stride(dtype))
        return cls(buf.ptr, shape, dtype, owner=buf)

    @classmethod
    def from_numpy(cls, arr: np.ndarray, dtype: Optional[str] = None, stream: Optional[Stream] = None) -> "Tensor":
        """Uploads `arr`. For bf16 pass uint16 bit patterns with dtype='bf16'."""
        if dtype is None:
            dtype = {np.dtype(np.float32): "f32", np.dtype(np.float16): "f16", np.dtype(np.int32): "i32"}[arr.dtype]
        host = _host_array(arr, dtype)
        t = cls.empty(host.shape, dtype)
        if host.nbytes:
            check(lib().popcorn_memcpy_h2d(t.ptr, host.ctypes.data, host.nbytes, _stream_handle(stream)))
        return t

    def numpy(self, stream: Optional[Stream] = None) -> np.ndarray:
        out = np.empty(self.shape, dtype=_NP[self.dtype])
        if out.nbytes:
            check(lib().popcorn_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes, _stream_handle(stream)))
        return out

    def copy_from(self, arr: np.ndarray, stream: Optional[Stream] = None) -> None:
        host = _host_array(arr, self.dtype)
        if host.nbytes > self.nbytes:
            raise ValueError("source larger than tensor")
        if host.nbytes:
            check(lib().popcorn_memcpy_h2d(self.ptr, host.ctypes.data, host.nbytes, _stream_handle(stream)))

    def fill_zero(self, stream: Optional[Stream] = None) -> None:
        check(lib().popcorn_memset(self.ptr, 0, self.nbytes, _stream_handle(stream)))

    def view(self, shape: Sequence[int], dtype: Optional[str] = None, offset_elements: int = 0) -> "Tensor":
        dt = dtype or self.dtype
        return Tensor(self.ptr + offset_elements * stride(self.dtype), shape, dt, owner=self.owner or self)

    @property
    def element_count(self) -> int:
        return int(np.prod(self.shape)) if self.shape else 1

    @property
    def nbytes(self) -> int:
        return self.element_count * stride(self.dtype)

    def desc(self) -> TensorDesc:
        d = TensorDesc()
        d.data = self.ptr
        d.dtype = DTYPES[self.dtype]
        d.rank = len(self.shape)
        for i, s in enumerate(self.shape):
            d.shape[i] = s
        return d

    def __repr__(self):
        return f"Tensor(shape={list(self.shape)}, dtype={self.dtype}, ptr=0x{self.ptr:x})"


def _d(t: Optional[Tensor]):
    return None if t is None else C.byref(t.desc())


# ---- block-affine quantized weights (AffineQuantizedTensor.swift:19-84) ----------

class AffineQuantizedTensor:
    """packed_values (u32 [..., out, in * bits / 32]), scales and optional biases
    ([..., out, in / group_size]) of a logical [..., out, in] tensor:
    w = q * scale + bias, values packed least-significant first
    (AffineQuantizationFormat.swift:24-30). Validated as the reference's init is."""

    def __init__(self, packed_values: Tensor, scales: Tensor, biases: Optional[Tensor], shape: Sequence[int],
                 bits: int = 4, group_size: int = 64):
        self.packed_values, self.scales, self.biases = packed_values, scales, biases
        self.shape, self.bits, self.group_size = list(shape), bits, group_size
        check(lib().popcorn_affine_quantized_validate(C.byref(self.desc())))

    @property
    def out_features(self) -> int:
        return self.shape[-2]

    @property
    def in_features(self) -> int:
        return self.shape[-1]

    def desc(self) -> _capi.AffineQuantizedDesc:
        d = _capi.AffineQuantizedDesc()
        d.packed_values = self.packed_values.desc()
        d.scales = self.scales.desc()
        if self.biases is not None:
            d.biases = self.biases.desc()
        d.rank = len(self.shape)
        for i, v in enumerate(self.shape):
            d.shape[i] = v
        d.bits, d.group_size = self.bits, self.group_size
        return d

    def tensors(self):
        return [t for t in (self.packed_values, self.scales, self.biases) if t is not None]


# ---- masks (AttentionMask.swift:17-41) -------------------------------------------

@dataclass(frozen=True)
class AttentionMask:
    kind: int = 0
    window: int = -1

    @staticmethod
    def causal_sliding_window(window: int) -> "AttentionMask":
        return AttentionMask(1, int(window))

    def desc(self) -> AttentionMaskDesc:
        return AttentionMaskDesc(self.kind, self.window if self.kind == 1 else -1)


AttentionMask.causal = AttentionMask(0)
AttentionMask.bidirectional = AttentionMask(2)


# ---- library (KernelLibrary.swift) -------------------------------------------------

class KernelFunction:
    def __init__(self, handle: int, name: str):
        self.handle = handle
        self.name = name

    def attributes(self) -> dict:
        a = _capi.FunctionAttrs()
        check(lib().popcorn_function_attributes(self.handle, C.byref(a)))
        return {f: getattr(a, f) for f, _ in a._fields_}


class KernelLibrary:
    """The gfx950 code objects (default: popcorn_amd/lib/kernels)."""

    def __init__(self, path: Optional[str] = None):
        h = C.c_void_p()
        check(lib().popcorn_library_load(path.encode() if path else None, C.byref(h)))
        self.handle = h.value

    def function(self, name: str) -> KernelFunction:
        """pipelineState(for:): cached; raises PopcornError(-1006) for an unknown name."""
        h = C.c_void_p()
        check(lib().popcorn_library_function(self.handle, name.encode(), C.byref(h)))
        return KernelFunction(h.value, name)

    @property
    def cached_function_count(self) -> int:
        return int(lib().popcorn_library_cached_function_count(self.handle))

    def layout(self, name: str) -> dict:
        """The kernel's parameter list from its code object: leading device
        pointers, then the byte size of each by-value block."""
        L = _capi.KernelLayout()
        check(lib().popcorn_function_layout(self.function(name).handle, C.byref(L)))
        return {"buffers": L.nbuffers, "constants": list(L.constant_sizes[:L.nconstants]),
                "max_threads": L.max_threads_per_block}

    def launch(self, name: str, grid, block, buffers: Sequence[int], constants: Sequence[bytes] = (),
               dynamic_lds: int = 0, stream: Optional[Stream] = None) -> None:
        """Raw launch: device pointers in order, then constants blocks by value."""
        fn = self.function(name)
        g = (C.c_uint32 * 3)(*grid)
        b = (C.c_uint32 * 3)(*block)
        bufs = (C.c_void_p * max(len(buffers), 1))(*buffers)
        keep = [C.create_string_buffer(c, len(c)) for c in constants]
        cptrs = (C.c_void_p * max(len(keep), 1))(*[C.cast(k, C.c_void_p) for k in keep])
        sizes = (C.c_size_t * max(len(keep), 1))(*[len(c) for c in constants])
        check(lib().popcorn_launch(_stream_handle(stream), fn.handle, g, b, bufs, len(buffers), cptrs, sizes,
                                   len(keep), dynamic_lds))

    def fill_normal(self, t: Tensor, seed: int, mean: float = 0.0, std: float = 1.0,
                    stream: Optional[Stream] = None) -> None:
        check(lib().popcorn_fill_normal(self.handle, _stream_handle(stream), t.ptr, DTYPES[t.dtype],
                                        t.element_count, seed, mean, std))

    def __del__(self):
        try:
            if self.handle:
                lib().popcorn_library_destroy(self.handle)
        except Exception:
            pass


# ---- scratch (KernelResources.swift) ---------------------------------------------------

class ScratchPool:
    """Best-fit pool of device buffers for one stream (a KernelScratchAllocator)."""

    def __init__(self):
        h = C.c_void_p()
        check(lib().popcorn_scratch_pool_create(C.byref(h)))
        self.handle = h.value

    def allocator(self) -> _capi.ScratchAllocatorDesc:
        a = _capi.ScratchAllocatorDesc()
        check(lib().popcorn_scratch_pool_allocator(self.handle, C.byref(a)))
        return a

    @property
    def nbytes(self) -> int:
        return int(lib().popcorn_scratch_pool_bytes(self.handle))

    def __del__(self):
        try:
            if self.handle:
                lib().popcorn_scratch_pool_destroy(self.handle)
        except Exception:
            pass


class KernelScratchAllocator:
    """Base for Python allocators: override borrow(length) -> (ptr, was_reused) and release(ptr)."""

    def borrow(self, length: int):
        raise NotImplementedError

    def release(self, ptr: int) -> None:
        pass

    def allocator(self) -> _capi.ScratchAllocatorDesc:
        def _borrow(ctx, length, out, reused):
            try:
                ptr, was_reused = self.borrow(int(length))
                out[0] = ptr
                if reused:
                    reused[0] = 1 if was_reused else 0
                return 0
            except Exception:
                return PopcornError.TENSOR_ALLOCATION_FAILED

        def _release(ctx, ptr):
            self.release(ptr)

        self._cb = (_capi.BORROW_FN(_borrow), _capi.RELEASE_FN(_release))
        return _capi.ScratchAllocatorDesc(None, self._cb[0], self._cb[1])


def code_object_layout(path: str, kernel: str) -> dict:
    """A kernel's parameter list read from a code-object file (no GPU needed)."""
    L = _capi.KernelLayout()
    check(lib().popcorn_code_object_layout(path.encode(), kernel.encode(), C.byref(L)))
    return {"buffers": L.nbuffers, "constants": list(L.constant_sizes[:L.nconstants]),
            "max_threads": L.max_threads_per_block}


def scratch_spec_byte_count(shape: Sequence[int], dtype: str) -> int:
    arr = (C.c_int64 * max(len(shape), 1))(*shape)
    return int(lib().popcorn_scratch_spec_byte_count(arr, len(shape), DTYPES[dtype]))


# ---- kernels (Kernel.swift + Kernels/*.swift) -----------------------------------------

class Kernel:
    """A validated operation descriptor; encode it with a KernelCommandEncoder."""

    def __init__(self, handle: int, refs: Iterable = ()):
        self.handle = handle
        self._refs = list(refs)  # tensors the descriptor points at

    def describe(self) -> str:
        buf = C.create_string_buffer(512)
        check(lib().popcorn_kernel_describe(self.handle, buf, 512))
        return buf.value.decode()

    @property
    def function_names(self):
        return self.describe().split(",")

    def __del__(self):
        try:
            if self.handle:
                lib().popcorn_kernel_destroy(self.handle)
        except Exception:
            pass


def _make(fn, *args, refs=()):
    h = C.c_void_p()
    check(fn(*args, C.byref(h)))
    return Kernel(h.value, refs)


class Kernels:
    """The operation descriptors of the decode hot path."""

    @staticmethod
    def route(query_len: int, head_dim: int, q_dtype: str = "bf16") -> str:
        r = lib().popcorn_flash_attention_route(query_len, head_dim, DTYPES[q_dtype])
        return {0: "plain", 1: "tiled", 2: "decoding"}[r]

    @staticmethod
    def FlashAttention(q: Tensor, k: Tensor, v: Tensor, into: Optional[Tensor] = None, *, scale: float,
                       mask: AttentionMask = AttentionMask(0), out: Optional[Tensor] = None,
                       batch: Optional[int] = None, query_heads: int = 0, kv_heads: int = 0, query_len: int = 0,
                       key_len: int = 0, head_dim: int = 0, key_capacity: int = 0,
                       position: Optional[Tensor] = None) -> Kernel:
        """FlashAttention(q:k:v:into:scale:mask:) (FlashAttention.swift:51-90), or with
        batch=... the explicit-dims init (:13-49) plus key_capacity / position."""
        o = into if into is not None else out
        refs = (q, k, v, o, position)
        if batch is None:
            return _make(lib().popcorn_kernel_flash_attention, _d(q), _d(k), _d(v), _d(o), scale, mask.desc(),
                         refs=refs)
        return _make(lib().popcorn_kernel_flash_attention_dims, _d(q), _d(k), _d(v), _d(o), batch, query_heads,
                     kv_heads, query_len, key_len, head_dim, scale, mask.desc(), key_capacity, _d(position),
                     refs=refs)

    @staticmethod
    def Matmul(a: Tensor, b, into: Tensor, transpose_b: bool = False, *, m: Optional[int] = None,
               k: int = 0, n: int = 0) -> Kernel:
        """Matmul(_:_:into:transposeB:) (Matmul.swift:68-93) or, with m=..., the dims init (:9-66);
        with an AffineQuantizedTensor b, Matmul(_:_:into:) (:99-130): c = a b^T."""
        if isinstance(b, AffineQuantizedTensor):
            return _make(lib().popcorn_kernel_matmul_quantized, _d(a), C.byref(b.desc()), _d(into),
                         refs=[a, into] + b.tensors())
        if m is None:
            return _make(lib().popcorn_kernel_matmul, _d(a), _d(b), _d(into), int(transpose_b), refs=(a, b, into))
        return _make(lib().popcorn_kernel_matmul_dims, _d(a), _d(b), _d(into), m, k, n, int(transpose_b),
                     refs=(a, b, into))

    @staticmethod
    def RMSNorm(x: Tensor, weight: Optional[Tensor] = None, into: Optional[Tensor] = None, *, axis: int = -1,
                eps: float, add_one_to_weight: bool = False, row_count: Optional[int] = None,
                hidden_size: int = 0) -> Kernel:
        """RMSNorm(_:weight:into:axis:eps:addOneToWeight:) (RMSNorm.swift:39-70), or with
        row_count=... the explicit init (:10-37)."""
        if row_count is None:
            return _make(lib().popcorn_kernel_rmsnorm, _d(x), _d(weight), _d(into), axis, eps,
                         int(add_one_to_weight), refs=(x, weight, into))
        return _make(lib().popcorn_kernel_rmsnorm_dims, _d(x), _d(weight), _d(into), row_count, hidden_size, eps,
                     int(add_one_to_weight), refs=(x, weight, into))

    @staticmethod
    def KVCacheWrite(source: Tensor, cache: Tensor, offset: int = 0, *, batch: Optional[int] = None,
                     kv_heads: int = 0, new_len: int = 0, max_len: int = 0, head_dim: int = 0,
                     position: Optional[Tensor] = None) -> Kernel:
        """KVCacheWrite(source:cache:offset:) (KVCacheWrite.swift:37-48) or the dims init (:7-35)."""
        if batch is None and position is None:
            return _make(lib().popcorn_kernel_kv_cache_write, _d(source), _d(cache), offset, refs=(source, cache))
        if batch is None:
            batch, kv_heads, new_len, head_dim = source.shape
            max_len = cache.shape[2]
        return _make(lib().popcorn_kernel_kv_cache_write_dims, _d(source), _d(cache), batch, kv_heads, new_len,
                     max_len, head_dim, offset, _d(position), refs=(source, cache, position))

    @staticmethod
    def GeluTanh(x: Tensor, into: Tensor) -> Kernel:
        return _make(lib().popcorn_kernel_gelu_tanh, _d(x), _d(into), refs=(x, into))

    @staticmethod
    def Mul(a: Tensor, b: Tensor, into: Tensor) -> Kernel:
        return _make(lib().popcorn_kernel_mul, _d(a), _d(b), _d(into), refs=(a, b, into))

    @staticmethod
    def Add(a: Tensor, b: Tensor, into: Tensor) -> Kernel:
        return _make(lib().popcorn_kernel_add, _d(a), _d(b), _d(into), refs=(a, b, into))

    @staticmethod
    def ScalarMul(x: Tensor, by: float, into: Tensor) -> Kernel:
        return _make(lib().popcorn_kernel_scalar_mul, _d(x), by, _d(into), refs=(x, into))

    @staticmethod
    def RopeBuildCosSin(positions: Tensor, inv_freq: Tensor, cos_out: Tensor, sin_out: Tensor, *,
                        attention_scaling: float = 1.0, seq_len: Optional[int] = None,
                        half_head_dim: int = 0) -> Kernel:
        """RopeBuildCosSin(positions:invFreq:cosOut:sinOut:attentionScaling:) (RopeBuildCosSin.swift:30-50),
        or with seq_len=... the explicit init (:8-28)."""
        refs = (positions, inv_freq, cos_out, sin_out)
        if seq_len is None:
            return _make(lib().popcorn_kernel_rope_build_cos_sin, _d(positions), _d(inv_freq), _d(cos_out),
                         _d(sin_out), attention_scaling, refs=refs)
        return _make(lib().popcorn_kernel_rope_build_cos_sin_dims, _d(positions), _d(inv_freq), _d(cos_out),
                     _d(sin_out), seq_len, half_head_dim, attention_scaling, refs=refs)

    @staticmethod
    def RopeApply(x: Tensor, cos: Tensor, sin: Tensor, into: Tensor, *, batch: Optional[int] = None,
                  seq_len: int = 0, head_count: int = 0, head_dim: int = 0) -> Kernel:
        """RopeApply(_:cos:sin:into:) (RopeApply.swift:46-60), or with batch=... the explicit init (:8-44)."""
        refs = (x, cos, sin, into)
        if batch is None:
            return _make(lib().popcorn_kernel_rope_apply, _d(x), _d(cos), _d(sin), _d(into), refs=refs)
        return _make(lib().popcorn_kernel_rope_apply_dims, _d(x), _d(cos), _d(sin), _d(into), batch, seq_len,
                     head_count, head_dim, refs=refs)

    @staticmethod
    def Transpose12(src: Tensor, into: Tensor, *, dims: Optional[Sequence[int]] = None) -> Kernel:
        """Transpose12(_:into:) (Transpose12.swift:27-35), or with dims=(d0, d1, d2, d3) the explicit init (:8-25)."""
        if dims is None:
            return _make(lib().popcorn_kernel_transpose12, _d(src), _d(into), refs=(src, into))
        d0, d1, d2, d3 = dims
        return _make(lib().popcorn_kernel_transpose12_dims, _d(src), _d(into), d0, d1, d2, d3, refs=(src, into))

    @staticmethod
    def GatedMLP(x: Tensor, norm_weight: Optional[Tensor], w_gate: Tensor, w_up: Tensor, w_down: Tensor,
                 into: Tensor, *, eps: float, add_one_to_weight: bool = False,
                 hidden: Optional[Tensor] = None) -> Kernel:
        """RMSNorm -> gate, up -> GeluTanh(gate) * up -> down (Gemma4TextInference.swift:416-429)."""
        return _make(lib().popcorn_kernel_gated_mlp, _d(x), _d(norm_weight), _d(w_gate), _d(w_up), _d(w_down),
                     _d(into), eps, int(add_one_to_weight), _d(hidden),
                     refs=(x, norm_weight, w_gate, w_up, w_down, into, hidden))

    @staticmethod
    def GatedMLPResidual(x_in: Tensor, delta: Tensor, w_post: Tensor, x_out: Tensor, norm_weight: Optional[Tensor],
                         w_gate: Tensor, w_up: Tensor, w_down: Tensor, into: Tensor, *, eps: float,
                         add_one_to_weight: bool = False, hidden: Optional[Tensor] = None) -> Kernel:
        """x_out = x_in + RMSNorm(delta) * w_post, then into = GatedMLP(x_out); with
        AffineQuantizedTensor weights the 4-bit form (delta, w_post, x_out may then be None)."""
        if isinstance(w_gate, AffineQuantizedTensor):
            qs = [w_gate.desc(), w_up.desc(), w_down.desc()]
            return _make(lib().popcorn_kernel_gated_mlp_residual_quantized, _d(x_in), _d(delta), _d(w_post),
                         _d(x_out), _d(norm_weight), *[C.byref(q) for q in qs], _d(into), eps, _d(hidden),
                         refs=[x_in, delta, w_post, x_out, norm_weight, into, hidden] + w_gate.tensors() +
                         w_up.tensors() + w_down.tensors())
        return _make(lib().popcorn_kernel_gated_mlp_residual, _d(x_in), _d(delta), _d(w_post), _d(x_out),
                     _d(norm_weight), _d(w_gate), _d(w_up), _d(w_down), _d(into), eps, int(add_one_to_weight),
                     _d(hidden), refs=(x_in, delta, w_post, x_out, norm_weight, w_gate, w_up, w_down, into, hidden))

    @staticmethod
    def DecodeMatvec(x: Tensor, weight: Tensor, into: Tensor, *, delta: Optional[Tensor] = None,
                     w_post: Optional[Tensor] = None, x_out: Optional[Tensor] = None, w_pre: Optional[Tensor] = None,
                     k_cache: Optional[Tensor] = None, v_cache: Optional[Tensor] = None,
                     position: Optional[Tensor] = None, q_rows: int = 0, eps: float = 1e-6) -> Kernel:
        """Decode matvec with the layer glue (popcorn_decode_matvec_args_t)."""
        qw = weight if isinstance(weight, AffineQuantizedTensor) else None
        ts = dict(x=x, delta=delta, w_post=w_post, x_out=x_out, w_pre=w_pre, weight=None if qw else weight,
                  out=into, k_cache=k_cache, v_cache=v_cache, position=position)
        descs = {n: (t.desc() if t is not None else None) for n, t in ts.items()}
        a = _capi.DecodeMatvecArgs()
        for n, d in descs.items():
            setattr(a, n, C.pointer(d) if d is not None else None)
        a.q_rows = q_rows
        a.eps = eps
        refs = list(ts.values())
        if qw is not None:
            qd = qw.desc()
            a.qweight = C.pointer(qd)
            refs += qw.tensors() + [qd]
        return _make(lib().popcorn_kernel_decode_matvec, C.byref(a), refs=refs)

    @staticmethod
    def DecodeAttention(qkv: Tensor, k_cache: Tensor, v_cache: Tensor, into: Tensor, position: Tensor, *,
                        query_heads: int, kv_heads: int, scale: float, q_norm: Optional[Tensor] = None,
                        k_norm: Optional[Tensor] = None, v_norm: bool = False, inv_freq: Optional[Tensor] = None,
                        rope_scaling: float = 1.0, eps: float = 1e-6,
                        mask: AttentionMask = AttentionMask(0)) -> Kernel:
        """One decode token's attention block with its per-head glue (popcorn_decode_attention_args_t):
        the reference's RMSNorm/RopeApply/Transpose12/KVCacheWrite/FlashAttention sequence
        (Gemma4TextInference.swift:352-399) as two dispatches."""
        ts = dict(qkv=qkv, k_cache=k_cache, v_cache=v_cache, out=into, position=position, q_norm=q_norm,
                  k_norm=k_norm, inv_freq=inv_freq)
        descs = {n: (t.desc() if t is not None else None) for n, t in ts.items()}
        a = _capi.DecodeAttentionArgs()
        for n, d in descs.items():
            setattr(a, n, C.pointer(d) if d is not None else None)
        a.v_norm = int(v_norm)
        a.query_heads = query_heads
        a.kv_heads = kv_heads
        a.eps = eps
        a.scale = scale
        a.rope_scaling = rope_scaling
        a.mask = mask.desc()
        return _make(lib().popcorn_kernel_decode_attention, C.byref(a), refs=list(ts.values()))

    @staticmethod
    def EmbeddingGather(ids: Tensor, table, into: Tensor) -> Kernel:
        """EmbeddingGather(ids:table:into:) (EmbeddingGather.swift:29-38, quantized table :45-88)."""
        if isinstance(table, AffineQuantizedTensor):
            return _make(lib().popcorn_kernel_embedding_gather_quantized, _d(ids), C.byref(table.desc()), _d(into),
                         refs=[ids, into] + table.tensors())
        return _make(lib().popcorn_kernel_embedding_gather, _d(ids), _d(table), _d(into), refs=(ids, table, into))

    @staticmethod
    def Argmax(x: Tensor, indices: Tensor) -> Kernel:
        return _make(lib().popcorn_kernel_argmax, _d(x), _d(indices), refs=(x, indices))

    @staticmethod
    def Custom(function_name: str, tensors: Sequence[Tensor], access: Sequence[int], constants: Sequence[bytes],
               grid, block) -> Kernel:
        """A caller-built DispatchKernel (Kernel.swift:54-70); access 1 read, 2 write, 3 both."""
        n = len(tensors)
        descs = (TensorDesc * max(n, 1))(*[t.desc() for t in tensors])
        acc = (C.c_uint8 * max(n, 1))(*access)
        keep = [C.create_string_buffer(c, len(c)) for c in constants]
        cptrs = (C.c_void_p * max(len(keep), 1))(*[C.cast(k, C.c_void_p) for k in keep])
        sizes = (C.c_size_t * max(len(keep), 1))(*[len(c) for c in constants])
        g = (C.c_uint32 * 3)(*grid)
        b = (C.c_uint32 * 3)(*block)
        return _make(lib().popcorn_kernel_custom, function_name.encode(), descs, acc, n, cptrs, sizes, len(keep),
                     g, b, refs=list(tensors))


# ---- encoder (KernelCommandEncoder.swift) ------------------------------------------------

class KernelCommandEncoder:
    """Encodes kernels in order on one stream; scratch from `scratch` (a ScratchPool
    or KernelScratchAllocator) or an internal pool."""

    def __init__(self, library: KernelLibrary, stream: Optional[Stream] = None, scratch=None):
        self.library = library
        self.stream = stream
        self._scratch = scratch
        alloc = scratch.allocator() if scratch is not None else None
        self._alloc = alloc
        h = C.c_void_p()
        check(lib().popcorn_encoder_create(library.handle, _stream_handle(stream),
                                           C.byref(alloc) if alloc is not None else None, C.byref(h)))
        self.handle = h.value

    def encode(self, *kernels) -> None:
        """encode(kernel), or several in order: the result-builder form encode { k1; k2 }."""
        flat = []
        for k in kernels:
            if isinstance(k, (list, tuple)):
                flat.extend(x for x in k if x is not None)
            elif k is not None:
                flat.append(k)
        if len(flat) == 1:
            check(lib().popcorn_encoder_encode(self.handle, flat[0].handle))
        elif flat:
            arr = (C.c_void_p * len(flat))(*[k.handle for k in flat])
            check(lib().popcorn_encoder_encode_all(self.handle, arr, len(flat)))

    def barrier(self) -> None:
        check(lib().popcorn_encoder_barrier(self.handle))

    def stats(self) -> dict:
        s = _capi.EncoderStats()
        check(lib().popcorn_encoder_stats(self.handle, C.byref(s)))
        return {"dispatches": s.dispatches, "hazards": s.hazards, "scratch_borrows": s.scratch_borrows}

    def close(self) -> None:
        if getattr(self, "handle", None):
            check(lib().popcorn_encoder_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
