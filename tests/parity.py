"""Parity checks shared by the GPU tests: a kernel output against the CPU oracle (oracle/).

Two bounds (oracle.within_tolerance, oracle.within_ulps):
* the north-star tolerance (rel-L2 <= 1e-2, max-abs <= 2e-2 on bf16 outputs, one ulp per
  bf16 rounding of the output's chain where an ulp exceeds 2e-2), always;
* a tight bound for kernels that compute the oracle's arithmetic in another fp32 summation
  order: a bounded fraction of outputs may differ, each by at most one bf16 ulp (at the
  largest magnitude along its rounding chain) plus c * 2^-24 * sum|x w| (cancellation).
"""
from __future__ import annotations

import numpy as np

from oracle import oracle

# Tight-bound parameters per kernel route (oracle.within_ulps): the bf16-decode routes (MFMA
# GEMM, skinny kernel) differ from the oracle only in fp32 summation order; the exact-weight
# GEMVs (1..8 rows) sum codes offset by 128 (x * (128 + q), then minus 128 * sum(x)), which
# carries about 7 fewer bits of the fp32 accumulator into each 32-weight group sum, hence a
# larger summation-error factor and flip allowance (measured 0.15-0.2 % of outputs).
ROUTES = {"bf16": dict(c=4.0, max_flip_fraction=1e-3), "exact": dict(c=64.0, max_flip_fraction=5e-3)}


def check(name, got, want, chain=(), term_sum=None, tight=True, route="bf16"):
    """North-star tolerance (rel-L2 <= 1e-2, max-abs <= 2e-2, one ulp per rounding of the chain
    where an ulp exceeds 2e-2) always; with ``tight`` also oracle.within_ulps for the route."""
    stats = oracle.compare_bf16(got, want)
    print(f"[{name}] {stats}", flush=True)
    assert oracle.within_tolerance(stats, got, want, chain=chain), (name, stats)
    if tight:
        ok, info = oracle.within_ulps(got, want, chain, term_sum, **ROUTES[route])
        print(f"[{name}] tight {info}", flush=True)
        assert ok, (name, info)
    return stats


def expect(x, w, bias=None):
    """(oracle output, its rounding chain, summation-error scale) for y = bf16(x w^T) (+ bias)."""
    want, chain = oracle.linear_reference_chain(x, w, oracle.bias_to_bf16(bias) if bias is not None else None)
    return want, chain, oracle.abs_term_sum(x, w)


def lora_term_sum(x, ads, m, n):
    """Per-output summation-error scale of the adapters that touch it (oracle.lora_abs_term_sum)."""
    s = np.zeros((m, n))
    for ad in ads:
        rb = ad.get("row_begin", 0)
        rc = m - rb if ad.get("row_count") is None else ad["row_count"]
        ob, oe = ad.get("out_begin", 0), ad.get("out_end") or n
        s[rb:rb + rc, ob:oe] += oracle.lora_abs_term_sum(x[rb:rb + rc], ad["a"], ad["b"], ad["scale"])
    return s


def check_lora(name, y, base, x, w, bias, ads, base_route="bf16"):
    """Runtime-LoRA output `y` whose base projection (same launches, no adapters, no bias) was
    `base`: (1) the base against the oracle GEMM, tight; (2) the adapters and the bias applied by
    the oracle on top of the kernel's own base bits, tight (only the adapters' fp32 sums
    differ); (3) end to end against the full oracle, north-star bound over the rounding chain."""
    m, n = y.shape
    bb = oracle.bias_to_bf16(bias) if bias is not None else None
    check(f"{name} base", base, *expect(x, w), route=base_route)
    want2, chain2 = oracle.linear_reference_chain(x, w, bb, ads, base_bf16=base)
    check(f"{name} adapters on kernel base", y, want2, chain2, lora_term_sum(x, ads, m, n))
    want3, chain3 = oracle.linear_reference_chain(x, w, bb, ads)
    check(f"{name} end to end", y, want3, chain3, tight=False)
