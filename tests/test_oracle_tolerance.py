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
    want = _outputs()
    assert oracle.within_ulps(want, want)[0]
    got = _step(want, np.arange(0, 20000, 1000), 1)  # 20 of 20000 (0.1 %) by one ulp
    ok, info = oracle.within_ulps(got, want)
    assert ok and info["differing"] == 20 and info["max_ulps_at_pre_bias"] == 1.0


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


def test_bias_cancellation_uses_pre_bias_ulp():
    """y_pre = 1.0 flips to the next bf16 value; a bias of -0.99 leaves a result whose own ulp
    is 2^7 times smaller: the flip is legal when the pre-bias magnitude is supplied, and the
    same difference without it is rejected."""
    pre = oracle.bf16_bits(np.array([1.0, 0.5], dtype=np.float32))
    bias = oracle.bf16_bits(np.array([-0.98828125, 0.25], dtype=np.float32))
    want = oracle.add_bias(pre, bias)
    got = oracle.add_bias(_step(pre, [0], 1), bias)
    assert oracle.within_ulps(got, want, pre, max_flip_fraction=0.5)[0]
    assert not oracle.within_ulps(got, want, None, max_flip_fraction=0.5)[0]


def test_dropped_rounding_step_fails():
    """A kernel that added the bias to the fp32 accumulator instead of to the rounded bf16
    value (one rounding instead of two) differs on a measurable fraction of outputs."""
    rng = np.random.default_rng(9)
    acc = (rng.standard_normal(20000) * 0.3).astype(np.float32)
    bias = oracle.bf16_bits((rng.standard_normal(20000) * 0.01).astype(np.float32))
    pre = oracle.bf16_bits(acc)
    want = oracle.add_bias(pre, bias)
    got = oracle.bf16_bits(acc + oracle.bf16_to_f32(bias))
    assert not oracle.within_ulps(got, want, pre)[0]
