"""GPU: the allocation-free entry point (tc_qlinear_forward_noalloc) against tc_qlinear_forward.

Each case makes two calls in a row through the C ABI, the second with a smaller input, and
compares every output with the allocating entry point's on the same inputs: bit for bit where
both split K the same way, else (fewer K slices because the partials exceed the fixed
scratch) within the tight summation-order bound of oracle.within_ulps (one bf16 ulp plus the
fp32 summation error of outputs whose terms cancel). The allocation-free
calls run first on each handle, so no per-handle workspace exists when they run.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu

Q4K, Q6K, Q8_0 = 12, 14, 8
SCRATCH = 32 << 20


@pytest.fixture(scope="module")
def mods():
    from turbocider_amd import _lib, gguf, qlinear
    return _lib, gguf, qlinear


def dev_weight(gguf, typ, n, k, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return gguf.quantize(torch.randn((n, k), generator=g, device="cuda") * 0.02, typ)


def dev_x(m, k, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)


def host(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def plan(_lib, typ, n, k, m):
    info = _lib.tc_qlinear_plan_info()
    _lib.call(_lib.lib().tc_qlinear_plan, typ, n, k, m, k, 0, C.byref(info))
    return info


def both(lin, x, adapters=()):
    y0 = lin(x, adapters, allocation_free=True)
    torch.cuda.synchronize()
    y1 = lin(x, adapters)
    torch.cuda.synchronize()
    return host(y0), host(y1)


@pytest.mark.parametrize("typ,n,k,ms", [
    (Q4K, 3584, 3584, (256, 100)),     # 128-row tiles, K split 7 ways (24.5 MiB of partials), then fewer
    (Q6K, 3072, 3072, (1024, 300)),    # config 1 shape on Q6_K: split 2 ways
    (Q4K, 3584, 3584, (64, 20)),       # skinny kernel, K split 4 ways
    (Q4K, 12288, 3072, (4096, 1)),     # north star (no split), then the one-row GEMV
])
def test_noalloc_matches_forward_same_split(mods, typ, n, k, ms):
    _lib, gguf, ql = mods
    g = torch.Generator(device="cuda").manual_seed(7)
    bias = torch.randn(n, generator=g, device="cuda") * 0.01
    lin = ql.QuantizedLinear(dev_weight(gguf, typ, n, k, 11), typ, n, k, bias)
    for i, m in enumerate(ms):
        assert plan(_lib, typ, n, k, m).workspace_bytes <= SCRATCH
        print(f"[noalloc] type={typ} n={n} k={k} m={m}", flush=True)
        a, b = both(lin, dev_x(m, k, 20 + i))
        assert np.array_equal(a, b), (m, int((a != b).sum()))


def test_noalloc_fewer_splits_when_partials_exceed_scratch(mods):
    """A long-K Q6_K projection (K = 18944, N = 2048) at M = 1024 and 700 (256-row tiles):
    tc_qlinear_forward splits K 8 and 10 ways into 64 and 60 MiB of partials, more than the
    32 MiB scratch; the allocation-free call uses fewer slices. Compared on sampled rows (tile
    edges and random rows; each output row depends only on its own activation row)."""
    _lib, gguf, ql = mods
    n, k = 2048, 18944
    blocks = dev_weight(gguf, Q6K, n, k, 12)
    lin = ql.QuantizedLinear(blocks, Q6K, n, k)
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks.cpu().numpy(), Q6K, n, k, dtype=oracle.DTYPE_BF16))
    for i, m in enumerate((1024, 700)):
        assert plan(_lib, Q6K, n, k, m).workspace_bytes > SCRATCH
        print(f"[noalloc fewer splits] m={m}", flush=True)
        x = dev_x(m, k, 30 + i)
        a, b = both(lin, x)
        rows = np.unique(np.concatenate([[0, 1, 255, 256, m - 1],
                                         np.random.default_rng(m).integers(0, m, 40)]))
        ok, info = oracle.within_ulps(a[rows], b[rows], (), oracle.abs_term_sum(host(x)[rows], wb))
        print(f"[noalloc fewer splits] m={m} {info}", flush=True)
        assert ok, info


def test_noalloc_runtime_lora(mods):
    """Per-image adapters (low rows in the scratch after the base launches' partials), then a
    smaller call with one adapter on a row segment and a partial output range."""
    _lib, gguf, ql = mods
    n, k = 3072, 3072
    g = torch.Generator(device="cuda").manual_seed(8)
    bias = torch.randn(n, generator=g, device="cuda") * 0.01
    lin = ql.QuantizedLinear(dev_weight(gguf, Q4K, n, k, 13), Q4K, n, k, bias)

    def adapter(r, rows, row_begin, out_begin, out_end, seed):
        gg = torch.Generator(device="cuda").manual_seed(seed)
        a = (torch.randn((r, k), generator=gg, device="cuda") / r).to(torch.bfloat16)
        b = (torch.randn((out_end - out_begin, r), generator=gg, device="cuda") * 0.01).to(torch.bfloat16)
        return ql.LoRAAdapter(a, b, 0.8, row_begin, rows, out_begin, out_end)

    calls = [(1024, [adapter(16, 512, 0, 0, n, 40), adapter(64, 512, 512, 0, n, 41)]),
             (600, [adapter(32, 300, 200, 512, 2048, 42)])]
    for m, ads in calls:
        assert plan(_lib, Q4K, n, k, m).workspace_bytes <= SCRATCH  # same K split on both entry points
        print(f"[noalloc lora] m={m} adapters={len(ads)}", flush=True)
        a, b = both(lin, dev_x(m, k, 50 + m), ads)
        assert np.array_equal(a, b), (m, int((a != b).sum()))


def test_noalloc_rejections(mods):
    _lib, gguf, ql = mods
    # A type other than Q4_K / Q5_K / Q6_K runs the library GEMM: rejected.
    raw = torch.zeros(256 * 34 // 32 * 4, dtype=torch.uint8, device="cuda")
    dense = ql.QuantizedLinear(raw, Q8_0, 4, 256)
    with pytest.raises(ql.QLinearError, match="Q4_K / Q5_K / Q6_K weights only"):
        dense(dev_x(2, 256, 60), allocation_free=True)
    # Adapter rows larger than the scratch at one K slice: rejected before any launch.
    n, k, m, r = 64, 256, 20000, 1024
    lin = ql.QuantizedLinear(dev_weight(gguf, Q4K, n, k, 14), Q4K, n, k)
    a = torch.zeros((r, k), dtype=torch.bfloat16, device="cuda")
    b = torch.zeros((n, r), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ql.QLinearError, match="fixed scratch"):
        lin(dev_x(m, k, 61), [ql.LoRAAdapter(a, b, 1.0)], allocation_free=True)
    # The same call through the allocating entry point is accepted.
    lin(dev_x(m, k, 61), [ql.LoRAAdapter(a, b, 1.0)])
    torch.cuda.synchronize()
