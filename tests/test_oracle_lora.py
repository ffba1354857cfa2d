"""CPU: pin the oracle's runtime-LoRA / bias sequence with the reference's fixed-bit KATs.

Expected bit patterns are the ones fixed by tests/native/native_lora_math_test.cpp:127-240
(fp32 low retained, adapter order, bias last, negative/zero scales, distinct A, rank-3
tail). Both oracle restatements are checked: the scalar C one (fp32 sums in index order,
like the reference spec) and the numpy one used by the GPU parity tests (float64 sums
rounded once to fp32). Also the stacked-alpha closed form delta = (x A^T) B^T * s * alpha/r
(tests/native/lora_joint_ab_test.cpp:22-24) and the scale rule of mlx.cpp:1442-1452.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle


def bf(values):
    return np.array(values, dtype=np.uint16)


def both(x, y, a, b, scale=1.0, **kw):
    """Apply one adapter with both restatements; they must agree on these exact cases."""
    s = oracle.lora_apply_scalar(x, y, a, b, scale, **kw)
    n = oracle.apply_adapter(y, x, a, b, scale, **kw)
    assert np.array_equal(s, n)
    return s


def test_fp32_low_is_retained():
    x = bf([[0x3F80, 0x3F80]])
    for rank in (16, 128):
        a = np.zeros((rank, 2), dtype=np.uint16)
        a[0, 0], a[0, 1] = 0x3F80, 0x3B80  # 1, 2^-8
        b = np.zeros((1, rank), dtype=np.uint16)
        b[0, 0] = 0x4380  # 256
        y = bf([[0xC380]])  # -256
        out = both(x, y, a, b)
        assert out[0, 0] == 0x3F80  # fp32 low 1.00390625 * 256 - 256 = 1


def test_adapter_order_and_bias_last():
    x, a = bf([[0x3F80]]), bf([[0x3F80]])
    small, large, combined = bf([[0x3B80]]), bf([[0x3C00]]), bf([[0x3C40]])
    one = bf([[0x3F80]])
    ordered = both(x, both(x, one, a, small), a, large)
    reversed_ = both(x, both(x, one, a, large), a, small)
    merged = both(x, one, a, combined)
    assert ordered[0, 0] == 0x3F81 and reversed_[0, 0] == 0x3F82 and merged[0, 0] == 0x3F82
    last = oracle.add_bias(both(x, one, a, large), small[0])
    first = oracle.add_bias(one, small[0])
    assert first[0, 0] == 0x3F80
    first = both(x, first, a, large)
    assert last[0, 0] == 0x3F82 and first[0, 0] == 0x3F81
    # the same through linear_reference: base y = 1 from a one-hot GEMM, adapter, then bias
    w = np.array([[1.0]], dtype=np.float32)
    y = oracle.linear_reference(x, w, small[0], [dict(a=a, b=large, scale=1.0)])
    assert y[0, 0] == 0x3F82


def test_negative_and_zero_scales():
    x, a, b = bf([[0x3F80]]), bf([[0x3F80]]), bf([[0x4000]])
    for scale, expected in ((-1.0, 0xBF80), (0.0, 0x3F80), (-0.0, 0x3F80)):
        assert both(x, bf([[0x3F80]]), a, b, scale)[0, 0] == expected


def test_distinct_a_factors():
    x = bf([[0x3F80, 0x3F80]])
    a1, a2, b = bf([[0x3F80, 0]]), bf([[0, 0x4000]]), bf([[0x3F80]])
    out = both(x, both(x, bf([[0]]), a1, b), a2, b)
    assert out[0, 0] == 0x4040  # 1 + 2 = 3


def test_rank3_tail_columns_and_untouched_padding():
    x = bf([0x3F80, 0x4000, 0xBF80, 0x4040, 0x4000, 0xC000]).reshape(3, 2)
    a = bf([0x3F80, 0, 0, 0x3F80, 0x3F80, 0xBF80]).reshape(3, 2)
    b = bf([0x40E0, 0x40E0, 0x40E0, 0xC080, 0x40A0, 0x40C0, 0x4000, 0, 0x3F80, 0, 0x3F80, 0xBF80,
            0x3F80, 0x3F80, 0]).reshape(5, 3)
    low = oracle.bf16_to_f32(x) @ oracle.bf16_to_f32(a).T
    assert np.array_equal(low.ravel(), np.array([1, 2, -1, -1, 3, -4, 2, -2, 4], dtype=np.float32))
    y = np.full((3, 5), 0x4180, dtype=np.uint16)  # 16
    out = both(x, y, a, b[2:5], out_begin=2, out_end=5)
    assert np.array_equal(out[:, 2:].ravel(), bf([0x4188, 0x4198, 0x4198, 0x4120, 0x41B8, 0x4190,
                                                   0x41C0, 0x4120, 0x4180]))
    assert (out[:, :2] == 0x4180).all()


def test_row_segments_leave_other_rows_bitwise_unchanged():
    rng = np.random.default_rng(3)
    x = oracle.bf16_bits(rng.standard_normal((6, 32)).astype(np.float32))
    y = oracle.bf16_bits(rng.standard_normal((6, 8)).astype(np.float32))
    y[0, 0] = 0x8000  # -0 must stay -0 outside the segment
    a = oracle.bf16_bits(rng.standard_normal((4, 32)).astype(np.float32))
    b = oracle.bf16_bits(rng.standard_normal((8, 4)).astype(np.float32))
    out = both(x, y, a, b, 0.75, row_begin=2, row_count=3)
    assert np.array_equal(out[[0, 1, 5]], y[[0, 1, 5]])
    assert not np.array_equal(out[2:5], y[2:5])


def test_stacked_alpha_closed_form():
    rng = np.random.default_rng(11)
    h, f, rank = 32, 64, 16
    a = oracle.bf16_bits((np.sin(np.arange(rank * f) * 0.013) * 0.025).astype(np.float32)).reshape(rank, f)
    b = oracle.bf16_bits((np.cos(np.arange(h * rank) * 0.017) * 0.03).astype(np.float32)).reshape(h, rank)
    x = oracle.bf16_bits(rng.standard_normal((5, f)).astype(np.float32))
    s = 0.5 * 4.0 / rank
    delta = oracle.lora_delta_f32(x, a, b) * np.float32(s)
    want = (oracle.bf16_to_f32(x).astype(np.float64) @ oracle.bf16_to_f32(a).T.astype(np.float64)
            @ oracle.bf16_to_f32(b).T.astype(np.float64)) * s
    assert np.linalg.norm(delta - want) / np.linalg.norm(want) < 1e-5


def _f32_round(v: Fraction) -> Fraction:
    """Round an exact rational to the nearest fp32 value, ties to even (IEEE 754 binary32:
    24-bit significand, minimum normal exponent -126, subnormals below it)."""
    if v == 0:
        return Fraction(0)
    sign, a = (-1 if v < 0 else 1), abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    scale = Fraction(2) ** (23 - e)
    q, r = divmod(a * scale, 1)
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and q % 2 == 1):
        q += 1
    out = sign * Fraction(q) / scale
    assert abs(out) < Fraction(2) ** 128, "fp32 overflow"
    return out


def _reference_scale(strength: float, rank: int, alpha: float | None) -> Fraction:
    """``float scale = strength; scale *= alpha / float(rank);`` (mlx.cpp:1442-1452) in exact
    rationals with one fp32 rounding per C operation; strength and alpha are fp32 values
    (LoRAAsset::strength is a float, core/contracts.hpp:17; alpha is read as float32)."""
    s = _f32_round(Fraction(strength))
    if alpha is None:
        return s
    ratio = _f32_round(_f32_round(Fraction(alpha)) / Fraction(rank))
    return _f32_round(s * ratio)


def _scale_triples():
    rng = np.random.default_rng(2024)
    strengths = [0.3, 0.75, 1.0, -0.25, 0.1, 1.3, 0.5, 0.9, 2.0 / 3.0, 1e-3]
    strengths += list(rng.uniform(0.5, 1.5, 11))
    alphas = [1.0, 3.0, 4.0, 8.0, 16.0, 32.0, 0.5, 6.0, 12.0, 7.5, 128.0, 1e-4]
    ranks = [1, 3, 7, 16, 20, 24, 48, 64, 96, 100, 128]
    for i, s in enumerate(strengths):
        for j, a in enumerate(alphas):
            yield float(s), ranks[(i + j) % len(ranks)], a
            yield float(s), ranks[(i * 3 + j * 5 + 1) % len(ranks)], a
    for s in strengths:
        yield float(s), 16, None


def test_scale_rule_matches_reference_fp32_steps():
    """lora_scale equals the reference's two fp32 roundings on >= 400 (strength, alpha, rank)
    triples, most with non-power-of-two alpha / rank ratios."""
    from turbocider_amd.qlinear import lora_scale
    triples = list(_scale_triples())
    assert len(triples) >= 400
    for s, r, a in triples:
        want = _reference_scale(s, r, a)
        got = lora_scale(s, r, a)
        assert Fraction(got) == want, (s, r, a, got, float(want))


def test_scale_rule_pin_rejects_one_rounding():
    """The pin tells the reference's two fp32 roundings from a single rounding of the exact
    (double-precision) product: on (0.3, alpha 1, rank 3) and (0.3, alpha 4, rank 7) the two
    differ, and lora_scale must give the two-rounding value."""
    from turbocider_amd.qlinear import lora_scale
    differ = 0
    for s, r, a in _scale_triples():
        one = _f32_round(Fraction(s) * Fraction(a) / Fraction(r)) if a is not None else None
        if one is not None and one != _reference_scale(s, r, a):
            differ += 1
    assert differ >= 20
    for s, r, a in [(0.3, 3, 1.0), (0.3, 7, 4.0)]:
        assert _f32_round(Fraction(s) * Fraction(a) / Fraction(r)) != _reference_scale(s, r, a)
        assert Fraction(lora_scale(s, r, a)) == _reference_scale(s, r, a)


def test_scale_rule_errors():
    from turbocider_amd.qlinear import QLinearError, lora_scale
    assert lora_scale(0.75, 16) == 0.75
    for bad in (float("inf"), float("nan")):
        with pytest.raises(QLinearError, match="LoRA alpha must be finite"):
            lora_scale(1.0, 4, bad)
    with pytest.raises(QLinearError, match="LoRA alpha must be finite"):
        lora_scale(1.0, 4, 1e39)  # finite double, not a finite float32
    with pytest.raises(QLinearError, match="LoRA effective scale must be finite"):
        lora_scale(3e38, 1, 4.0)
