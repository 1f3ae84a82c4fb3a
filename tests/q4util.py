"""Test helpers for block-affine 4-bit weights: an MLX-style group quantizer
(min/max per group of 64, scale = (max - min) / 15, bias = min, both stored
bf16) and the packing of AffineQuantizationFormat.swift:25-29 (value i of a
row in bits 4 (i % 8) of word i / 8). The reference ships no quantizer; these
only make realistic inputs."""
import numpy as np

import oracle as O


def pack_q4(q):
    """q uint [N, K] in 0..15 -> u32 [N, K / 8], lowest index in the lowest bits."""
    q = np.asarray(q, np.uint64)
    N, K = q.shape
    shifts = (4 * np.arange(8, dtype=np.uint64))[None, None, :]
    return (q.reshape(N, K // 8, 8) << shifts).sum(axis=-1).astype(np.uint32)


def unpack_q4(words, K):
    w = np.asarray(words, np.uint32)
    N = w.shape[0]
    shifts = (4 * np.arange(8, dtype=np.uint32))[None, None, :]
    return ((w[:, :, None] >> shifts) & 15).reshape(N, K)


def quantize_q4(w, group=64, bias=True):
    """w f32 [N, K] -> (packed u32 [N, K/8], scales, biases f32 [N, K/group] with
    bf16 values, q [N, K])."""
    w = np.asarray(w, np.float32)
    N, K = w.shape
    g = w.reshape(N, K // group, group)
    lo, hi = g.min(axis=-1), g.max(axis=-1)
    if not bias:
        lo = np.zeros_like(lo)
        hi = np.abs(g).max(axis=-1)
    scale = (hi - lo) / 15.0
    scale[scale == 0] = 1.0
    scale = O.round_to(scale.astype(np.float32), O.BF16)
    b = O.round_to(lo.astype(np.float32), O.BF16)
    q = np.clip(np.rint((g - b[..., None]) / scale[..., None]), 0, 15).astype(np.uint32).reshape(N, K)
    return pack_q4(q), scale, (b if bias else None), q


def dequantize_q4(q, scales, biases, group=64):
    """f32 values q * s + b, rounded as a float32 multiply then add."""
    N, K = q.shape
    s = np.repeat(np.asarray(scales, np.float32), group, axis=1)
    b = np.repeat(np.asarray(biases, np.float32), group, axis=1) if biases is not None else np.float32(0)
    return (q.astype(np.float32) * s + b).astype(np.float32)
