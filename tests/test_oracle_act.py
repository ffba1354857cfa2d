"""CPU: the oracle's output activations (oracle.act_reference) pinned independently of their
own formulas.

* Against torch's float64 GELU (approximate="tanh") and SiLU on every finite bf16 value of
  magnitude below 64: an independent implementation of the same functions.
* Odd-part identities that a wrong sign, constant or operand would break:
  gelu(z) - gelu(-z) = z and silu(z) - silu(-z) = z; gelu(0) = silu(0) = 0; gelu(z) -> z and
  -> 0 at the ends.
* The float64 -> bf16 rounding against exact rational arithmetic on ties and near-ties.
* A planted mistake (the cubic coefficient 0.044715 replaced by 0.04715) fails the torch check.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import oracle


def _all_bf16(limit=64.0):
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    v = oracle.bf16_to_f32(bits)
    keep = np.isfinite(v) & (np.abs(v) < limit)
    return bits[keep], v[keep].astype(np.float64)


def test_gelu_and_silu_match_torch_float64():
    """torch evaluates GELU in the tanh form, which loses relative precision where 1 + tanh(u)
    cancels; above z = -5 it keeps better than 1e-9, far below a bf16 ulp."""
    _, z = _all_bf16()
    t = torch.from_numpy(z)
    s_ref = torch.nn.functional.silu(t).numpy()
    assert np.allclose(oracle.silu_f64(z), s_ref, rtol=1e-13, atol=1e-300)
    zg = z[z >= -5.0]
    g_ref = torch.nn.functional.gelu(torch.from_numpy(zg), approximate="tanh").numpy()
    assert np.allclose(oracle.gelu_tanh_f64(zg), g_ref, rtol=1e-9, atol=1e-300)


def test_gelu_negative_tail_follows_its_asymptote():
    """Below z = -5: gelu(z) = z e^{2u} / (1 + e^{2u}) -> z e^{2u}, relative gap e^{2u}."""
    _, z = _all_bf16()
    zt = z[z < -5.0]
    u = np.sqrt(2.0 / np.pi) * (zt + 0.044715 * zt ** 3)
    lead = zt * np.exp(2.0 * u)
    g = oracle.gelu_tanh_f64(zt)
    assert np.all(np.abs(g - lead) <= np.abs(lead) * (np.exp(2.0 * u) + 1e-14) + 1e-300)


def test_planted_gelu_constant_is_caught():
    _, z = _all_bf16()
    z = z[z >= -5.0]
    u = np.sqrt(2.0 / np.pi) * (z + 0.04715 * z ** 3)
    bad = z / (1.0 + np.exp(-2.0 * u))
    ref = torch.nn.functional.gelu(torch.from_numpy(z), approximate="tanh").numpy()
    assert not np.allclose(bad, ref, rtol=1e-9, atol=1e-300)


def test_odd_part_identities_and_limits():
    _, z = _all_bf16(16.0)
    assert np.allclose(oracle.gelu_tanh_f64(z) - oracle.gelu_tanh_f64(-z), z, rtol=1e-14, atol=1e-14)
    assert np.allclose(oracle.silu_f64(z) - oracle.silu_f64(-z), z, rtol=1e-14, atol=1e-14)
    assert oracle.gelu_tanh_f64(np.array([0.0]))[0] == 0.0 and oracle.silu_f64(np.array([0.0]))[0] == 0.0
    assert oracle.gelu_tanh_f64(np.array([40.0]))[0] == 40.0 and abs(oracle.gelu_tanh_f64(np.array([-40.0]))[0]) < 1e-300
    assert oracle.silu_f64(np.array([-1000.0]))[0] == 0.0


def _bf16_exact(v: Fraction) -> int:
    """RNE of a rational to bf16 bits by exact arithmetic (positive normal values)."""
    e = 0
    while v >= 2:
        v /= 2
        e += 1
    while v < 1:
        v *= 2
        e -= 1
    scaled = v * 128  # 7 fraction bits
    q, r = divmod(scaled.numerator, scaled.denominator)
    half = Fraction(scaled.denominator, 2)
    rem = Fraction(r)
    if rem > half or (rem == half and q & 1):
        q += 1
    if q == 256:
        q, e = 128, e + 1
    return ((e + 127) << 7) | (q - 128)


def test_f64_to_bf16_rounding_is_single_rne():
    rng = np.random.default_rng(7)
    vals = []
    for _ in range(300):
        b = int(rng.integers(0x3000, 0x5000))
        lo = Fraction(float(oracle.bf16_to_f32(np.array([b], np.uint16))[0]))
        hi = Fraction(float(oracle.bf16_to_f32(np.array([b + 1], np.uint16))[0]))
        mid = (lo + hi) / 2
        eps = (hi - lo) / (1 << 30)  # below float32's resolution: double rounding would tie
        vals += [mid, mid + eps, mid - eps, lo + (hi - lo) / 3]
    got = oracle.bf16_bits_from_f64(np.array([float(v) for v in vals]))
    want = [_bf16_exact(Fraction(float(v))) for v in vals]
    assert list(map(int, got)) == want


def test_act_reference_layout():
    rng = np.random.default_rng(3)
    pre = oracle.bf16_bits(rng.standard_normal((3, 8)).astype(np.float32))
    h = oracle.act_reference(pre, oracle.ACT_SILU_GLU)
    z = oracle.bf16_to_f32(pre).astype(np.float64)
    assert h.shape == (3, 4)
    assert np.array_equal(h, oracle.bf16_bits_from_f64(oracle.silu_f64(z[:, ::2]) * z[:, 1::2]))
    with pytest.raises(ValueError):
        oracle.act_reference(pre, 9)


def _decimal_bf16(val):
    """Exact RNE of a Decimal to bf16 bits by bracketing (positive or negative, normal range)."""
    from decimal import Decimal
    a = abs(val)
    f = float(a)
    lo = int(np.array([f], np.float32).view(np.uint32)[0] >> 16)
    while Decimal(float(oracle.bf16_to_f32(np.array([lo], np.uint16))[0])) > a:
        lo -= 1
    while Decimal(float(oracle.bf16_to_f32(np.array([lo + 1], np.uint16))[0])) <= a:
        lo += 1
    lo_v = Decimal(float(oracle.bf16_to_f32(np.array([lo], np.uint16))[0]))
    hi_v = Decimal(float(oracle.bf16_to_f32(np.array([lo + 1], np.uint16))[0]))
    mid = (lo_v + hi_v) / 2
    bits = lo + 1 if (a > mid or (a == mid and lo & 1)) else lo
    return bits | (0x8000 if val < 0 else 0)


def test_act_reference_rounds_the_exact_value():
    """act_reference against a 60-digit decimal evaluation of every output of a sample that
    includes gates large enough for sigmoid to round to 1 in float64 (g u then often sits
    exactly halfway between two bf16 values, and the exact value just below it)."""
    from decimal import Decimal, localcontext
    rng = np.random.default_rng(11)
    g = oracle.bf16_bits(np.concatenate([rng.standard_normal(600) * 3, rng.uniform(37, 80, 600)]).astype(np.float32))
    u = oracle.bf16_bits((rng.standard_normal(1200) * 3).astype(np.float32))
    pre = np.stack([g, u], 1).reshape(1, -1)
    got = oracle.act_reference(pre, oracle.ACT_SILU_GLU).reshape(-1)
    gz = oracle.act_reference(g[:600].reshape(1, -1), oracle.ACT_GELU_TANH).reshape(-1)
    pi = Decimal("3.14159265358979323846264338327950288419716939937510582097494")
    with localcontext() as ctx:
        ctx.prec = 60
        for i in range(1200):
            dg = Decimal(float(oracle.bf16_to_f32(g[i:i + 1])[0]))
            du = Decimal(float(oracle.bf16_to_f32(u[i:i + 1])[0]))
            val = dg * du / (1 + (-dg).exp())
            want = 0 if val == 0 else _decimal_bf16(val)
            assert (int(got[i]) & 0x7FFF) == (want & 0x7FFF) == 0 or int(got[i]) == want, (i, dg, du)
        for i in range(600):
            d = Decimal(float(oracle.bf16_to_f32(g[i:i + 1])[0]))
            val = d / (1 + (-(2 * (2 / pi).sqrt() * (d + Decimal("0.044715") * d ** 3))).exp())
            want = 0 if val == 0 else _decimal_bf16(val)
            assert (int(gz[i]) & 0x7FFF) == (want & 0x7FFF) == 0 or int(gz[i]) == want, (i, d)
    # The tie case that float64 alone rounds the wrong way: g = 72, u = 1.46875.
    pair = oracle.bf16_bits(np.array([[72.0, 1.46875]], np.float32))
    assert int(oracle.act_reference(pair, oracle.ACT_SILU_GLU)[0, 0]) == 0x42D3
