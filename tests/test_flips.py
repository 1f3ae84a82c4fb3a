"""CPU checks of the rounding-outcome helpers the GPU tests judge by: the
composition they rebuild equals the oracle's own gated MLP, a kernel whose
norm scale sits a few f32 ulps off the oracle's passes, and planted mistakes
fail against every outcome."""
import numpy as np
import pytest

import flips
import oracle as O
from conftest import assert_out

H, FF = 512, 2048


def _data(tag, seed=0):
    x = O.round_to(O.normal(seed, (H,), std=2.0), tag)
    nw = O.normal(seed + 1, (H,), mean=1.0, std=0.1)
    wg, wu = (O.round_to(O.normal(seed + s, (FF, H), std=0.02), tag) for s in (2, 3))
    wd = O.round_to(O.normal(seed + 4, (H, FF), std=0.02), tag)
    return x, nw, wg, wu, wd


@pytest.mark.parametrize("tag", [O.BF16, O.F16, O.F32])
def test_mlp_from_normed_is_the_oracle_gated_mlp(tag):
    x, nw, wg, wu, wd = _data(tag)
    h_ref, out_ref = O.gated_mlp(x, nw, 1e-6, wg, wu, wd, inter_tag=tag)
    n = O.round_to(O.rmsnorm(x, nw, 1e-6), tag)
    h, out = flips.mlp_from_normed(n, wg, wu, wd, tag)
    np.testing.assert_array_equal(h, h_ref)
    np.testing.assert_array_equal(out, out_ref)


def _kernel_like(x, nw, wg, wu, wd, tag, scale_err, w=None):
    """The composition with the norm scale off by `scale_err` (relative)."""
    tf = O.rmsnorm(x, nw if w is None else w, 1e-6).astype(np.float64)
    n = O.round_to((tf * (1 + scale_err)).astype(np.float32), tag)
    return flips.mlp_from_normed(n, wg, wu, wd, tag)[1]


@pytest.mark.parametrize("tag,name", [(O.BF16, "bf16"), (O.F16, "f16")])
@pytest.mark.parametrize("seed", range(6))
def test_scale_within_noise_passes(tag, name, seed):
    x, nw, wg, wu, wd = _data(tag, 10 * seed)
    cands = [flips.mlp_from_normed(n, wg, wu, wd, tag)[1] for n in flips.norm_candidates(x, nw, 1e-6, tag)]
    for err in (-2.0 ** -20, -2.0 ** -22, 0.0, 2.0 ** -21, 2.0 ** -20):
        flips.assert_any(O.round_to(_kernel_like(x, nw, wg, wu, wd, tag, err), tag), cands, 2e-3, name, "noise")


def test_plain_rounding_is_a_candidate():
    x, nw, *_ = _data(O.BF16, 3)
    plain = O.round_to(O.rmsnorm(x, nw, 1e-6), O.BF16)
    assert any(np.array_equal(c, plain) for c in flips.norm_candidates(x, nw, 1e-6, O.BF16))


def test_some_seed_has_several_outcomes():
    # the helper is not vacuous: midpoints do occur at these sizes
    counts = [len(flips.norm_candidates(O.round_to(O.normal(s, (2304,), std=2.0), O.BF16),
                                        O.normal(s + 1, (2304,), mean=1.0, std=0.1), 1e-6, O.BF16))
              for s in range(20)]
    assert max(counts) > 1 and min(counts) >= 1


@pytest.mark.parametrize("mistake", ["no_norm_weight", "transposed_down", "gate_up_swapped_in_gelu", "scale_1e-2"])
def test_planted_mistakes_fail(mistake):
    tag = O.BF16
    x, nw, wg, wu, wd = _data(tag, 7)
    cands = [flips.mlp_from_normed(n, wg, wu, wd, tag)[1] for n in flips.norm_candidates(x, nw, 1e-6, tag)]
    if mistake == "no_norm_weight":
        bad = _kernel_like(x, nw, wg, wu, wd, tag, 0.0, w=np.ones_like(nw))
    elif mistake == "transposed_down":
        n = O.round_to(O.rmsnorm(x, nw, 1e-6), tag)
        h, _ = flips.mlp_from_normed(n, wg, wu, wd, tag)
        bad = O.matmul(h, wd.reshape(FF, H), 1, FF, H, False).ravel()
    elif mistake == "gate_up_swapped_in_gelu":
        bad = flips.mlp_from_normed(O.round_to(O.rmsnorm(x, nw, 1e-6), tag), wu, wg, wd, tag)[1]
    else:
        bad = _kernel_like(x, nw, wg, wu, wd, tag, 1e-2)
    with pytest.raises(AssertionError):
        flips.assert_any(O.round_to(bad, tag), cands, 2e-3, "bf16", mistake)


def test_residual_candidates_match_reference_composition():
    tag = O.BF16
    x_in = O.round_to(O.normal(1, (H,)), tag)
    d = O.round_to(O.normal(2, (H,), std=3.0), tag)
    wp = O.normal(3, (H,), mean=1.0, std=0.1)
    plain = O.round_to(O.add(x_in, O.round_to(O.rmsnorm(d, wp, 1e-6), tag)), tag)
    cands = flips.residual_candidates(x_in, d, wp, 1e-6, tag)
    assert any(np.array_equal(c, plain) for c in cands)
    assert_out(plain, cands[0], 2e-3, "bf16", "candidates are one ulp apart at most", half_ulps=4)
