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


# ---- exact hidden-vector outcomes -------------------------------------------
# A gate or up dot product summed in another f32 order differs from the
# oracle's by rounding errors of its partial sums, which grow like
# ||terms||_2: about sqrt(K) 2^-24 ||terms||_2 for a K-term sum in random
# order, K 2^-26 ||terms||_2 below (sqrt(K) / 4 times that: 12 at K 2304), and
# the kernel's GELU-tanh (hardware exp2) differs from the oracle's libm tanh
# by a few ulps of 0.5 v (1 + tanh), which cancels for negative v. Every
# 16-bit value a g, u or a = round(gelu(g)) can take inside those windows is
# a candidate; h = round(a * u) is then computed exactly as the reference
# stores it, and the kernel's h must equal one candidate bit for bit. An
# element whose window reaches across zero (|g| or |u| below its window, a
# few in ten thousand) takes the windows' propagated bound instead.
SUM_WINDOW = 2.0 ** -26
GELU_WINDOW = 2.0 ** -21
MAX_STEPS = 4


def _ordered(v, tag):
    """16-bit values -> integers in value order (sign-magnitude patterns)."""
    b = O.to_bits(np.asarray(v, np.float32), tag).astype(np.int64)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def _from_ordered(o, tag):
    b = np.where(o < 0, (-o) | 0x8000, o).astype(np.uint16)
    return O.from_bits(b, tag)


def _rounding_span(lo, hi, tag):
    """The tag values round(v) takes for v in [lo, hi], elementwise: a
    [MAX_STEPS, n] array padded with NaN, and the mask of elements whose span
    is longer (left out)."""
    a = _ordered(O.round_to(np.asarray(lo, np.float32), tag), tag)
    b = _ordered(O.round_to(np.asarray(hi, np.float32), tag), tag)
    wide = b - a >= MAX_STEPS
    out = np.full((MAX_STEPS,) + a.shape, np.nan, np.float32)
    for k in range(MAX_STEPS):
        o = a + k
        out[k] = np.where((o <= b) & ~wide, _from_ordered(np.minimum(o, b), tag), np.nan)
    return out, wide


class HiddenOutcomes:
    """Exact h outcomes for gate and up f32 sums g32, u32 of K terms whose
    2-norms are g_norm, u_norm."""

    def __init__(self, g32, u32, g_norm, u_norm, K, tag):
        self.tag = tag
        wg = K * SUM_WINDOW * np.asarray(g_norm, np.float64)
        wu = K * SUM_WINDOW * np.asarray(u_norm, np.float64)
        gs, gwide = _rounding_span(g32 - wg, g32 + wg, tag)
        us, uwide = _rounding_span(u32 - wu, u32 + wu, tag)
        out, wide = [], gwide | uwide
        for g in gs:
            g0 = np.nan_to_num(g)
            gl = O.gelu_tanh(g0).astype(np.float64)
            w = GELU_WINDOW * (np.abs(gl) + 0.5 * np.abs(g0))
            As, awide = _rounding_span(gl - w, gl + w, tag)
            wide |= awide & ~np.isnan(g)
            for a in As:
                for u in us:
                    h = O.round_to(O.mul(np.nan_to_num(a), np.nan_to_num(u)), tag)
                    out.append(np.where(np.isnan(g) | np.isnan(a) | np.isnan(u), np.nan, h))
        self.candidates = np.stack(out)
        self.wide = wide
        # for the wide elements: the reference composition and the bound the
        # windows propagate to (|dg| |u| / 2 + |gelu| |du| + two 16-bit steps)
        g16, u16 = O.round_to(g32.astype(np.float32), tag), O.round_to(u32.astype(np.float32), tag)
        self.ref = O.round_to(O.mul(O.round_to(O.gelu_tanh(g16), tag), u16), tag).astype(np.float64)
        self.bound = 0.6 * (wg + np.abs(g32) * 2.0 ** -7) * np.abs(u32) + np.abs(gl) * (wu + np.abs(u32) * 2.0 ** -7) \
            + 2 * np.abs(self.ref) * 2.0 ** -7

    def check(self, actual, what):
        a = np.asarray(actual, np.float32).ravel()
        ok = (self.candidates == a[None, :]).any(axis=0)
        ok[self.wide] = np.abs(a[self.wide] - self.ref[self.wide]) <= self.bound[self.wide]
        if not np.all(ok):
            bad = np.flatnonzero(~ok)
            i = bad[0]
            c = self.candidates[:, i]
            raise AssertionError(f"{what}: {bad.size}/{a.size} elements match no exact outcome; first at {i}: "
                                 f"{a[i]!r} vs {sorted(set(c[~np.isnan(c)].tolist()))} (wide: {bool(self.wide[i])})")


def dense_hidden(n, w_gate, w_up, tag):
    """HiddenOutcomes for dense weights [F, H] on the normed vector n."""
    F, H = w_gate.shape
    n = np.asarray(n, np.float32).ravel()
    g32 = O.matmul(n, w_gate, 1, H, F, True).ravel().astype(np.float64)
    u32 = O.matmul(n, w_up, 1, H, F, True).ravel().astype(np.float64)
    n2 = n.astype(np.float64) ** 2
    return HiddenOutcomes(g32, u32, np.sqrt(w_gate.astype(np.float64) ** 2 @ n2),
                          np.sqrt(w_up.astype(np.float64) ** 2 @ n2), H, tag)
