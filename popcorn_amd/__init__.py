"""popcorn_amd — the MI355X (gfx950) build of Popcorn's decode hot path.

HIP kernels for gfx950 (popcorn_amd/csrc/kernels) loaded as code objects by a
C++ runtime with a C ABI (include/popcorn_hip.h, popcorn_amd/lib/
libpopcorn_amd.so); this package is the Python mirror of the reference's
Swift API over that ABI.
"""
from ._capi import LIB_PATH, KERNEL_DIR  # noqa: F401
from .runtime import (  # noqa: F401
    AffineQuantizedTensor,
    UncachedBuffer,
    attention_pair_flags,
    AttentionMask,
    DeviceBuffer,
    Event,
    Kernel,
    KernelCommandEncoder,
    KernelFunction,
    KernelLibrary,
    Kernels,
    KernelScratchAllocator,
    PopcornError,
    ScratchPool,
    Stream,
    Tensor,
    check,
    device_count,
    device_info,
    lib,
    code_object_layout,
    scratch_spec_byte_count,
    stride,
    synchronize,
)
