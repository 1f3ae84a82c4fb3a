"""Rounding-outcome sets for checks downstream of an RMSNorm.

A kernel sums x^2 in another order than the oracle, so its f32 norm scale
differs from the oracle's in the last bits. Every element of the normed
vector is rounded to 16 bits with that one scale, so the elements that lie
within that noise of a rounding midpoint can round the other way, all
decided by where the kernel's scale falls. This module lists the distinct
16-bit normed vectors a scale within SCALE_NOISE (relative) of the oracle's
produces; a GPU result is held to the full bar against the composition run
on one of them. Everything away from a midpoint is fixed, so the set is
small (usually one to three vectors) and a real error (a dropped weight, a
wrong epsilon, a transposed operand) still fails against all of them.
"""
import numpy as np

import oracle as O
from conftest import assert_out

# ~2e-6 relative: a few f32 ulps, the spread of a few-thousand-term sum of
# squares taken in different orders (measured: under 2^-20 on gfx950).
SCALE_NOISE = 2.0 ** -19
MAX_AMBIGUOUS = 32


def scaled_candidates(tf, tag, noise=SCALE_NOISE, s_lo=1.0, s_hi=1.0):
    """The distinct round(tf * s) for s in [s_lo (1 - noise), s_hi (1 + noise)]."""
    tf = np.asarray(tf, np.float64)
    if tag == O.F32:  # no 16-bit store: the f32 bar covers the scale noise
        return [tf.astype(np.float32)]
    a, b = s_lo * (1 - noise), s_hi * (1 + noise)
    lo = O.round_to((tf * a).astype(np.float32), tag).astype(np.float64)
    hi = O.round_to((tf * b).astype(np.float32), tag).astype(np.float64)
    amb = np.flatnonzero(lo != hi)
    assert amb.size <= MAX_AMBIGUOUS, f"{amb.size} elements near a midpoint"
    # element i flips where tf_i * s crosses the midpoint of its two roundings
    thresholds = np.sort((lo[amb] + hi[amb]) / 2 / tf[amb])
    edges = np.concatenate([[a], thresholds, [b]])
    points = (edges[:-1] + edges[1:]) / 2
    out, seen = [], set()
    for s in points:
        c = O.round_to((tf * s).astype(np.float32), tag)
        key = c.tobytes()
        if key not in seen:
            seen.add(key)
            out.append(c)
    return out


def norm_candidates(x, w, eps, tag, add_one=False):
    """16-bit RMSNorm(x) * w outcomes (RMSNorm.metal:32-40) over the scale noise.

    The window spans the reference loop's scale (a sequential f32 sum of
    squares, the oracle's) and the exact one (the sum in float64): over a few
    thousand terms the sequential f32 sum can itself sit a few 2^-20 from the
    exact sum, and a kernel summing in a shallower order lands near the exact
    scale."""
    x = np.asarray(x, np.float32)
    acc = np.float32(0)
    for v in x.ravel():
        acc = np.float32(acc + np.float32(v * v))
    s32 = 1.0 / np.sqrt(np.float32(acc / np.float32(x.size) + np.float32(eps)))
    s64 = 1.0 / np.sqrt(np.sum(x.astype(np.float64) ** 2) / x.size + eps)
    r = float(s64) / float(s32)
    return scaled_candidates(O.rmsnorm(x, w, eps, add_one), tag, s_lo=min(1.0, r), s_hi=max(1.0, r))


def residual_candidates(x_in, delta, w_post, eps, tag):
    """round(x_in + round(RMSNorm(delta) * w_post)) outcomes."""
    return [O.round_to(O.add(x_in, t), tag) for t in norm_candidates(delta, w_post, eps, tag)]


def assert_any(actual, candidates, eps, out_dtype, what, half_ulps=1):
    """`actual` within the bar of at least one candidate expectation."""
    errors = []
    for c in candidates:
        try:
            assert_out(actual, c, eps, out_dtype, what, half_ulps=half_ulps)
            return
        except AssertionError as e:
            errors.append(str(e))
    raise AssertionError(f"{what}: no rounding outcome of the norm scale matches ({len(candidates)} tried): "
                         + " | ".join(errors))


def mlp_from_normed(n, w_gate, w_up, w_down, tag):
    """Gate, up, GeluTanh(gate) * up, down on an already normed vector, every
    intermediate stored in `tag` (Gemma4TextInference.swift:416-429); returns
    (hidden, f32 output)."""
    F, H = w_gate.shape
    g = O.round_to(O.matmul(n, w_gate, 1, H, F, True).ravel(), tag)
    u = O.round_to(O.matmul(n, w_up, 1, H, F, True).ravel(), tag)
    h = O.round_to(O.mul(O.round_to(O.gelu_tanh(g), tag), u), tag)
    return h, O.matmul(h, w_down, 1, F, H, True).ravel()
