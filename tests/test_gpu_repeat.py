"""GPU: repeated calls of the kernels whose loads are ordered by hand-counted waits.

k_skinny and k_gemm wait for their activation DMA with explicit `s_waitcnt vmcnt(N)` counts
that assume the exact issue order of the loads after it, and k_gemm keeps a tile's output
stores in flight under the next tile's first chunks. A wrong count, or a compiler that moves
a load across the ordering fences, reads an LDS buffer before its DMA has landed: the output
then differs from call to call. Each case here runs the same projection many times into an
output buffer that is overwritten with a NaN pattern before every call, and requires every
call to return the first call's bits (the first call is checked against the oracle by the
other GPU tests for these shapes). Cases cover the skinny kernel (Q4_K / Q6_K, split and
unsplit K, fused segments) and the GEMM (persistent 256-row tiles with several tiles per
workgroup, 128-row split tiles, a grouped launch).
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

Q4K, Q6K = 12, 14
REPEATS = 25


@pytest.fixture(scope="module")
def mods():
    from turbocider_amd import gguf, qlinear
    return gguf, qlinear


def weight(gguf, typ, n, k, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return gguf.quantize(torch.randn((n, k), generator=g, device="cuda") * 0.02, typ)


def act(m, k, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)


def poison(*ts):
    for t in ts:
        t.view(torch.int16).fill_(0x7FC1)  # a bf16 NaN no kernel produces


def repeat_equal(name, run, outs):
    """Run `run()` REPEATS times into `outs` (poisoned before each call); every call must
    return the first call's bits."""
    poison(*outs)
    run()
    torch.cuda.synchronize()
    first = [o.clone() for o in outs]
    for i in range(REPEATS - 1):
        poison(*outs)
        run()
        torch.cuda.synchronize()
        for j, (o, f) in enumerate(zip(outs, first)):
            same = torch.equal(o.view(torch.int16), f.view(torch.int16))
            assert same, (name, i + 1, j, int((o.view(torch.int16) != f.view(torch.int16)).sum()))
    for f in first:
        assert not torch.isnan(f.float()).any(), name


@pytest.mark.parametrize("typ,m,n,k", [
    (Q4K, 64, 18944, 3584),   # skinny, 296 tiles, unsplit
    (Q6K, 64, 3584, 18944),   # skinny, K split 4 ways
    (Q4K, 33, 3584, 3584),    # skinny, 3 row groups, K split
    (Q6K, 47, 12288, 1280),   # skinny, prefetch clamped at the slice end
])
def test_skinny_repeated_calls_identical(mods, typ, m, n, k):
    gguf, ql = mods
    lin = ql.QuantizedLinear(weight(gguf, typ, n, k, 1), typ, n, k)
    x = act(m, k, 2)
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    print(f"[repeat skinny] type={typ} {m}x{n}x{k}", flush=True)
    repeat_equal(f"skinny t{typ} {m}x{n}x{k}", lambda: lin(x, out=y), [y])


def test_skinny_fused_segments_repeated_calls_identical(mods):
    gguf, ql = mods
    n, k, m = 3584, 3584, 64
    lins = [ql.QuantizedLinear(weight(gguf, Q4K, n, k, 10 + i), Q4K, n, k) for i in range(3)]
    x = act(m, k, 13)
    ys = [torch.empty((m, n), dtype=torch.bfloat16, device="cuda") for _ in lins]
    print("[repeat skinny fused q/k/v]", flush=True)
    repeat_equal("skinny fused", lambda: ql.forward_many(lins, x, outs=ys), ys)


@pytest.mark.parametrize("typ,m,n,k", [
    (Q4K, 4096, 12288, 3072),  # north star: 768 tiles, 3 per persistent workgroup (after-full waits)
    (Q6K, 4132, 4096, 4096),   # 256-row tiles + a 36-row tail on the skinny kernel
    (Q4K, 1024, 3072, 3072),   # 128-row tiles, K split 2 ways
    (Q6K, 256, 3584, 18944),   # 128-row tiles, long K split
])
def test_gemm_repeated_calls_identical(mods, typ, m, n, k):
    gguf, ql = mods
    g = torch.Generator(device="cuda").manual_seed(3)
    lin = ql.QuantizedLinear(weight(gguf, typ, n, k, 4), typ, n, k, torch.randn(n, generator=g, device="cuda") * 0.01)
    x = act(m, k, 5)
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    print(f"[repeat gemm] type={typ} {m}x{n}x{k}", flush=True)
    repeat_equal(f"gemm t{typ} {m}x{n}x{k}", lambda: lin(x, out=y), [y])


def test_grouped_gemm_repeated_calls_identical(mods):
    gguf, ql = mods
    n, k = 3072, 3072
    l0 = ql.QuantizedLinear(weight(gguf, Q6K, n, k, 20), Q6K, n, k)
    l1 = ql.QuantizedLinear(weight(gguf, Q6K, n, k, 21), Q6K, n, k)
    x0, x1 = act(1024, k, 22), act(256, k, 23)
    ys = [torch.empty((1024, n), dtype=torch.bfloat16, device="cuda"),
          torch.empty((256, n), dtype=torch.bfloat16, device="cuda")]
    print("[repeat grouped gemm]", flush=True)
    repeat_equal("grouped", lambda: ql.forward_group([l0, l1], [x0, x1], outs=ys), ys)
