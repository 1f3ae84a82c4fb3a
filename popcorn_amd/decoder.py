"""The batch-1 greedy decode loop (include/popcorn_decoder.h) from Python."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, fields
from typing import Optional

import numpy as np

from . import _capi
from ._capi import DTYPE_NAMES
from .runtime import KernelLibrary, Stream, Tensor, check, lib


@dataclass
class DecoderConfig:
    layers: int = 26
    hidden: int = 2304
    query_heads: int = 8
    kv_heads: int = 4
    head_dim: int = 256
    ffn: int = 9216
    vocab: int = 256000
    max_seq: int = 4352
    eps: float = 1e-6
    attn_scale: float = 1.0 / 16.0
    history_len: int = 4352
    graph_steps: int = 1
    attention_block: int = 0      # 1: per-head q/k/v RMSNorm and RoPE (a real attention block)
    rope_theta: float = 10000.0
    weight_bits: int = 16         # 4: block-affine 4-bit weights (group 64, bf16 scales and biases)

    def c(self) -> _capi.DecoderConfig:
        return _capi.DecoderConfig(*[getattr(self, f.name) for f in fields(self)])


GEMMA2_2B = DecoderConfig()


class Decoder:
    """Owns the device state of a Gemma-shaped decoder; `step` enqueues tokens."""

    def __init__(self, library: KernelLibrary, stream: Stream, config: DecoderConfig = GEMMA2_2B):
        self.library, self.stream, self.config = library, stream, config
        h = C.c_void_p()
        cfg = config.c()
        check(lib().popcorn_decoder_create(library.handle, stream.handle, C.byref(cfg), C.byref(h)))
        self.handle = h.value

    def randomize(self, seed: int = 0) -> None:
        check(lib().popcorn_decoder_randomize(self.handle, seed))

    def tensor(self, name: str, layer: int = 0) -> Tensor:
        d = _capi.TensorDesc()
        check(lib().popcorn_decoder_tensor(self.handle, name.encode(), layer, C.byref(d)))
        return Tensor(d.data, [d.shape[i] for i in range(d.rank)], DTYPE_NAMES[d.dtype], owner=self)

    def reset(self, token: int, position: int) -> None:
        check(lib().popcorn_decoder_reset(self.handle, token, position))

    def step(self, steps: int = 1, use_graph: bool = True) -> None:
        check(lib().popcorn_decoder_step(self.handle, steps, int(use_graph)))

    def read(self):
        t, p = C.c_int32(), C.c_int32()
        check(lib().popcorn_decoder_read(self.handle, C.byref(t), C.byref(p)))
        return t.value, p.value

    def history(self, start: int, count: int) -> np.ndarray:
        h = self.tensor("history").numpy(self.stream)
        idx = (np.arange(start, start + count) % h.size)
        return h[idx]

    def describe(self):
        buf = C.create_string_buffer(1 << 16)
        n = C.c_int32()
        check(lib().popcorn_decoder_describe(self.handle, buf, 1 << 16, C.byref(n)))
        return buf.value.decode().split(","), n.value

    def step_bytes(self, position: int) -> int:
        return int(lib().popcorn_decoder_step_bytes(self.handle, position))

    def time_kernel_in_step(self, function_name: str, steps: int = 4):
        """(mean ms per launch, launches) of one kernel inside `steps` eager decode steps (advances the position)."""
        ms, n = C.c_float(), C.c_int32()
        check(lib().popcorn_decoder_time_kernel_in_step(self.handle, function_name.encode(), steps, C.byref(ms),
                                                        C.byref(n)))
        return ms.value, n.value

    def time_kernel(self, function_name: str, reps: int = 5):
        """(mean ms per launch, launches) of one kernel of the step, launched alone."""
        ms, n = C.c_float(), C.c_int32()
        check(lib().popcorn_decoder_time_kernel(self.handle, function_name.encode(), reps, C.byref(ms), C.byref(n)))
        return ms.value, n.value

    def close(self) -> None:
        if getattr(self, "handle", None):
            check(lib().popcorn_decoder_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
