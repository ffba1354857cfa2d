"""CPU: the parity bounds themselves (oracle.within_tolerance, oracle.within_ulps).

The tight bound must accept what a different fp32 summation order can produce (a rare
one-ulp rounding flip, also after a bias that cancels most of the value) and reject the
plausible kernel mistakes the loose north-star bound lets through: a small shift of many
outputs, a two-ulp error, a dropped rounding step.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle


def _outputs(n=20000, seed=5):
    rng = np.random.default_rng(seed)
    return oracle.bf16_bits(rng.standard_normal(n).astype(np.float32))


def _step(bits: np.ndarray, idx, ulps: int) -> np.ndarray:
    """Move the selected bf16 values by `ulps` units in the last place (away from zero)."""
    out = bits.copy()
    out[idx] = (out[idx].astype(np.int32) + ulps).astype(np.uint16)
    return out


def test_identical_and_rare_flips_pass():
    """20 of 20000 outputs (0.1 %) one ulp off: allowed."""
    want = _outputs()
    assert oracle.within_ulps(want, want)[0]
    got = _step(want, np.arange(0, 20000, 1000), 1)
    ok, info = oracle.within_ulps(got, want)
    assert ok and info["differing"] == 20 and info["max_diff_over_bound"] == 1.0


def test_many_small_shifts_fail_tight_but_pass_loose():
    """A bug shifting 1 % of outputs by one ulp each passes the north-star tolerance
    (max-abs 2e-2) but not the tight bound."""
    want = _outputs()
    got = _step(want, np.arange(0, 20000, 100), 1)
    stats = oracle.compare_bf16(got, want)
    assert oracle.within_tolerance(stats, got, want)
    assert not oracle.within_ulps(got, want)[0]


def test_two_ulp_error_fails():
    want = _outputs()
    small = np.flatnonzero(np.abs(oracle.bf16_to_f32(want)) < 1.0)[:1]
    got = _step(want, small, 2)
    stats = oracle.compare_bf16(got, want)
    assert oracle.within_tolerance(stats, got, want)  # loose bound accepts it
    assert not oracle.within_ulps(got, want)[0]


def test_tie_after_bias_doubles_a_flip():
    """A one-ulp flip before the bias becomes two ulps after it when y + bias is a tie: allowed
    with the chain, rejected without it (a single rounding)."""
    pre = oracle.bf16_bits(np.array([0.4375], dtype=np.float32))           # 0x3EE0
    bias = oracle.bf16_bits(np.array([2.0 ** -10], dtype=np.float32))     # half an ulp at 0.4375
    want = oracle.add_bias(pre, bias)                                      # tie -> even: 0.4375
    got = oracle.add_bias(_step(pre, [0], 1), bias)                        # tie -> even: 0.4375 + 2 ulps
    assert int(got.flat[0]) - int(want.flat[0]) == 2
    assert oracle.within_ulps(got, want, (pre,), max_flip_fraction=1.0)[0]
    assert not oracle.within_ulps(got, want, (), max_flip_fraction=1.0)[0]


def test_bias_cancellation_uses_pre_bias_ulp():
    """y_pre = 1.0 flips to the next bf16 value; a bias of -0.99 leaves a result whose own ulp
    is 2^7 times smaller: the flip is legal when the pre-bias magnitude is supplied, and the
    same difference without it is rejected."""
    pre = oracle.bf16_bits(np.array([1.0, 0.5], dtype=np.float32))
    bias = oracle.bf16_bits(np.array([-0.98828125, 0.25], dtype=np.float32))
    want = oracle.add_bias(pre, bias)
    got = oracle.add_bias(_step(pre, [0], 1), bias)
    assert oracle.within_ulps(got, want, (pre,), max_flip_fraction=0.5)[0]
    assert not oracle.within_ulps(got, want, (), max_flip_fraction=0.5)[0]


def test_dropped_rounding_step_fails():
    """A kernel that added the bias to the fp32 accumulator instead of to the rounded bf16
    value (one rounding instead of two) differs on a measurable fraction of outputs."""
    rng = np.random.default_rng(9)
    acc = (rng.standard_normal(20000) * 0.3).astype(np.float32)
    bias = oracle.bf16_bits((rng.standard_normal(20000) * 0.01).astype(np.float32))
    pre = oracle.bf16_bits(acc)
    want = oracle.add_bias(pre, bias)
    got = oracle.bf16_bits(acc + oracle.bf16_to_f32(bias))
    assert not oracle.within_ulps(got, want, (pre,))[0]


def test_cancellation_allowance_scales_with_term_sum():
    """An output whose terms cancel (|y| far below sum|x w|) may differ by a few fp32 units of
    the term sum, not by a bf16 ulp of its own tiny magnitude; the same difference on an
    output with a small term sum is rejected. Checked on a real fp32 GEMM against the oracle:
    every output of a float32 BLAS product is within the bound."""
    rng = np.random.default_rng(12)
    m, n, k = 64, 512, 2048
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wb = oracle.bf16_to_f32(oracle.bf16_bits(w))
    x = oracle.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    want, chain = oracle.linear_reference_chain(x, wb)
    got = oracle.bf16_bits(oracle.bf16_to_f32(x) @ wb.T)   # another fp32 summation order
    S = oracle.abs_term_sum(x, wb)
    assert oracle.within_ulps(got, want, chain, S)[0]
    # Planted: a near-zero output moved by 1e-3 is far outside c * 2^-24 * S.
    idx = np.unravel_index(np.argmin(np.abs(oracle.bf16_to_f32(want))), want.shape)
    bad = got.copy()
    bad[idx] = oracle.bf16_bits(np.array([oracle.bf16_to_f32(want[idx]) + 1e-3], dtype=np.float32))[0]
    assert not oracle.within_ulps(bad, want, chain, S)[0]


def test_chain_tolerance_allows_one_ulp_per_rounding():
    """at |y| in [2, 4) (ulp 2^-6 > 2e-2 / 2) an output two roundings deep may
    differ by two ulps (0.03125 > 2e-2), one only by one."""
    want = _outputs()
    want[0] = oracle.bf16_bits(np.array([3.0], dtype=np.float32))[0]
    got = _step(want, [0], 2)
    stats = oracle.compare_bf16(got, want)
    assert not oracle.within_tolerance(stats, got, want)
    assert oracle.within_tolerance(stats, got, want, chain=(want,))
