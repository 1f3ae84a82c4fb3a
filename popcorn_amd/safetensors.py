"""safetensors archives and the weight loader of the reference's example app,
over the native reader (include/popcorn_safetensors.h).

`SafeTensors` stands for the archive of the MTLSafeTensors dependency the
reference opens (Examples/GemmaCLI/Sources/GemmaCLI/Gemma4TextInference.swift:22);
`WeightLoader` mirrors Gemma4WeightLoader.swift:14-120: MLX vs Transformers
name prefixes, and a weight `<name>.weight` read as block-affine quantized
when `<name>.scales` and `<name>.biases` are present and a quantization
config is given.
"""
from __future__ import annotations

import ctypes as C
from typing import Dict, List, Optional, Tuple, Union

import numpy as np

from . import _capi
from ._capi import DTYPE_NAMES
from .runtime import AffineQuantizedTensor, PopcornError, Stream, Tensor, _NP, check, lib


class SafeTensors:
    """A mapped, validated safetensors file."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib().popcorn_safetensors_open(path.encode(), C.byref(h)))
        self.handle = h.value
        self.path = path
        self._infos: Dict[str, _capi.SafetensorsInfo] = {}
        for i in range(lib().popcorn_safetensors_count(self.handle)):
            info = _capi.SafetensorsInfo()
            check(lib().popcorn_safetensors_info(self.handle, i, C.byref(info)))
            self._infos[info.name.decode()] = info

    @property
    def names(self) -> List[str]:
        return list(self._infos)

    def __contains__(self, name: str) -> bool:
        return name in self._infos

    def info(self, name: str) -> Tuple[str, List[int]]:
        """(dtype, shape) of a tensor; dtype is the archive's name ("BF16", "U32", ...)."""
        i = self._find(name)
        return i.dtype_name.decode(), [i.shape[d] for d in range(i.rank)]

    def dtype(self, name: str) -> Optional[str]:
        """The tensor data type ("bf16", "u32", ...), None for dtypes without one (F64, F8_*)."""
        t = self._find(name).dtype
        return DTYPE_NAMES[t] if t >= 0 else None

    def metadata(self, key: str) -> str:
        buf = C.create_string_buffer(1 << 16)
        check(lib().popcorn_safetensors_metadata(self.handle, key.encode(), buf, len(buf)))
        return buf.value.decode()

    def read(self, name: str) -> np.ndarray:
        """A host copy (bf16 as uint16 bits)."""
        i = self._find(name)
        dt = self.dtype(name)
        if dt is None:
            raise PopcornError(-1010, f"safetensors dtype {i.dtype_name.decode()} has no tensor data type here")
        out = np.empty([i.shape[d] for d in range(i.rank)], _NP[dt])
        check(lib().popcorn_safetensors_read(self.handle, name.encode(), out.ctypes.data, out.nbytes))
        return out

    def tensor(self, name: str, stream: Optional[Stream] = None) -> Tensor:
        """A device copy in a fresh 256-byte aligned buffer (SafeTensors.tensor(named:))."""
        i = self._find(name)
        dt = self.dtype(name)
        if dt is None:
            raise PopcornError(-1010, f"safetensors dtype {i.dtype_name.decode()} has no tensor data type here")
        t = Tensor.empty([i.shape[d] for d in range(i.rank)], dt)
        check(lib().popcorn_safetensors_upload(self.handle, name.encode(), t.ptr, t.nbytes,
                                               stream.handle if stream is not None else None))
        return t

    def _find(self, name: str) -> _capi.SafetensorsInfo:
        if name not in self._infos:
            info = _capi.SafetensorsInfo()
            check(lib().popcorn_safetensors_find(self.handle, name.encode(), C.byref(info)))  # raises
        return self._infos[name]

    def close(self) -> None:
        if getattr(self, "handle", None):
            check(lib().popcorn_safetensors_close(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class WeightLoader:
    """Gemma4WeightLoader.swift:14-120 over a SafeTensors archive.

    quantization: None (dense only) or {"bits": b, "group_size": g}, the
    config's top-level quantization block."""

    def __init__(self, archive: SafeTensors, quantization: Optional[dict] = None):
        self.archive = archive
        self.quantization = quantization
        names = archive.names
        # Gemma4WeightLoader.swift:21-29
        if any(n.startswith("language_model.model.") for n in names):
            self.language_model_prefix = "language_model.model"
        elif any(n.startswith("model.language_model.") for n in names):
            self.language_model_prefix = "model.language_model"
        else:
            raise PopcornError(-1100, "Could not find Gemma language model weights in archive.")

    def qualify(self, relative: str) -> str:
        return f"{self.language_model_prefix}.{relative}"

    def layer_prefix(self, index: int) -> str:
        return self.qualify(f"layers.{index}")

    def linear(self, name: str, stream: Optional[Stream] = None) -> Union[Tensor, AffineQuantizedTensor]:
        """Dense `<name>.weight`, or the quantized triplet (Gemma4WeightLoader.swift:48-53)."""
        q = self._maybe_quantized(name, stream)
        return q if q is not None else self.archive.tensor(f"{name}.weight", stream)

    def embedding(self, name: str, stream: Optional[Stream] = None) -> Union[Tensor, AffineQuantizedTensor]:
        q = self._maybe_quantized(name, stream)
        return q if q is not None else self.archive.tensor(f"{name}.weight", stream)

    def _maybe_quantized(self, name: str, stream) -> Optional[AffineQuantizedTensor]:
        # Gemma4WeightLoader.swift:80-119
        if self.quantization is None:
            return None
        w, s, b = f"{name}.weight", f"{name}.scales", f"{name}.biases"
        if not (w in self.archive and s in self.archive and b in self.archive):
            return None
        if self.archive.dtype(w) != "u32":
            raise PopcornError(-1100, f"Expected U32 packed weights for {w}, got {self.archive.info(w)[0]}.")
        packed = self.archive.tensor(w, stream)
        bits = int(self.quantization["bits"])
        out_features, packed_inner = packed.shape[0], packed.shape[1]
        return AffineQuantizedTensor(packed, self.archive.tensor(s, stream), self.archive.tensor(b, stream),
                                     [out_features, packed_inner * (32 // bits)], bits=bits,
                                     group_size=int(self.quantization["group_size"]))
