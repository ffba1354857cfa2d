"""GPU: Q5_K projections on the hand-written kernels (the MFMA dequant-GEMM and the one-row
GEMV), against the oracle.

Q5_K (type 13, 176-byte blocks: d, dmin, 12 scale bytes, a 32-byte high-bit plane, 128 qs
bytes; gguf_decode.cpp:77-90) is read in place by both kernels: no bf16 copy, no library GEMM.
Weights are random blocks under small finite scales, so every code (0..31) and every high
bit pattern occurs. Checks:
* one-hot activations through the GEMM return the bf16-decoded weights bit for bit (every
  tile shape: 32-, 64-, 128- and 256-row tiles);
* the GEMM against the bf16-decode oracle (tight summation-order bound), unsplit, split K and
  with bias; 2..64 rows on the small tiles;
* the one-row GEMV against the exact-weight oracle, with ragged N, an odd super-block count,
  fused segments (forward_many) and the gated activation epilogue;
* the 2..8-row GEMV against the exact-weight oracle (ragged N, an odd super-block count, bias,
  fused segments);
* the skinny kernel (9..64 rows, and forced at 2..8): one-hot exactness, the bf16-decode oracle
  with and without K split and bias, fused segments and the gated activation epilogue.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from parity import check, expect
from test_gpu_qlinear import activations, canonical, dense_type_payload, from_dev_bf16, run_linear, to_dev_bf16
from test_plan import GEMM, GEMV1, GEMV8, SKINNY, plan

pytestmark = pytest.mark.gpu

Q5K = 13


@pytest.fixture(scope="module")
def ql():
    from turbocider_amd import qlinear
    return qlinear


def q5k(n, k, seed):
    return dense_type_payload(Q5K, n, k, np.random.default_rng(seed))


def decoded(raw, n, k, bf16=True):
    if bf16:
        return oracle.bf16_to_f32(oracle.decode_matrix(raw, Q5K, n, k, dtype=oracle.DTYPE_BF16))
    return oracle.decode_matrix(raw, Q5K, n, k)


@pytest.mark.parametrize("m", [20, 60, 512, 4096])
def test_q5k_gemm_one_hot_exact(ql, m):
    """Rows of the identity (repeated to m rows) through the GEMM give the bf16 weights."""
    n, k = 300, 512
    raw = q5k(n, k, 1)
    x = np.zeros((m, k), dtype=np.uint16)
    x[np.arange(m), np.arange(m) % k] = 0x3F80
    print(f"[q5k one-hot] m={m}", flush=True)
    y = run_linear(ql, raw, Q5K, n, k, x, path=1)
    want = oracle.decode_matrix(raw, Q5K, n, k, dtype=oracle.DTYPE_BF16).T[np.arange(m) % k]
    assert np.array_equal(canonical(y), canonical(want))


@pytest.mark.parametrize("m,n,k,split", [(300, 768, 512, None), (256, 512, 4096, True), (1024, 6144, 512, False),
                                         (5, 1000, 768, None), (40, 2048, 1024, None)])
def test_q5k_gemm_matches_oracle(ql, m, n, k, split):
    path = 1 if m <= 64 else 0  # 2..64 rows run the skinny kernel unless the GEMM is forced
    st, info, _ = plan(Q5K, n, k, m, path=path)
    assert st == 0 and info.kernel == GEMM
    if split is not None:
        assert (info.workspace_bytes > 0) == split
    raw = q5k(n, k, 10 + m)
    x = activations(m, k, 11 + m)
    bias = (np.random.default_rng(12).standard_normal(n) * 0.1).astype(np.float32)
    print(f"[q5k gemm] m={m} n={n} k={k}", flush=True)
    y = run_linear(ql, raw, Q5K, n, k, x, bias=bias, path=path)
    check(f"q5k gemm m={m}", y, *expect(x, decoded(raw, n, k), bias))


@pytest.mark.parametrize("n,k", [(4096, 1024), (300, 768), (18432, 3072)])
def test_q5k_gemv_matches_oracle(ql, n, k):
    """M = 1 on the one-row GEMV: exact fp32 weights (ragged N = 300, odd block count at
    K = 768, the adaLN shape)."""
    st, info, _ = plan(Q5K, n, k, 1)
    assert st == 0 and info.kernel == GEMV1
    raw = q5k(n, k, 20 + n)
    x = activations(1, k, 21)
    bias = (np.random.default_rng(22).standard_normal(n) * 0.1).astype(np.float32)
    print(f"[q5k gemv] n={n} k={k}", flush=True)
    y = run_linear(ql, raw, Q5K, n, k, x, bias=bias)
    check(f"q5k gemv n={n}", y, *expect(x, decoded(raw, n, k, bf16=False), bias), route="exact")


def test_q5k_gemv_fused_segments_and_activation(ql):
    n, k = 1536, 1024
    raws = [q5k(n, k, 30 + i) for i in range(3)]
    lins = [ql.QuantizedLinear(torch.from_numpy(r).cuda(), Q5K, n, k) for r in raws]
    x = activations(1, k, 33)
    print("[q5k gemv] forward_many", flush=True)
    ys = ql.forward_many(lins, to_dev_bf16(x))
    torch.cuda.synchronize()
    for i, (y, r) in enumerate(zip(ys, raws)):
        check(f"q5k segment {i}", from_dev_bf16(y), *expect(x, decoded(r, n, k, bf16=False)), route="exact")
    # The gated activation epilogue on a Q5_K gate_up binding at one row.
    W = ql.Weights()
    W.bind_glu("gu", torch.from_numpy(raws[0]).cuda(), torch.from_numpy(raws[1]).cuda(), Q5K, n, k)
    xd = to_dev_bf16(x)
    pre = from_dev_bf16(W._linears["gu"](xd))
    h = from_dev_bf16(W.project_act(xd, "gu", "silu_glu"))
    want = oracle.act_reference(pre, oracle.ACT_SILU_GLU)
    assert np.count_nonzero(h != want) <= oracle.allowed_differing(h.size, 1e-3)


@pytest.mark.parametrize("m", [2, 16, 40, 64])
def test_q5k_skinny_one_hot_exact(ql, m):
    """Rows of the identity through the skinny kernel give the bf16-decoded weights (the fifth
    code bit of every group, both nibbles, every lane's 8-column piece)."""
    n, k = 200, 512
    raw = q5k(n, k, 40 + m)
    x = np.zeros((m, k), dtype=np.uint16)
    x[np.arange(m), (7 * np.arange(m)) % k] = 0x3F80
    print(f"[q5k skinny one-hot] m={m}", flush=True)
    y = run_linear(ql, raw, Q5K, n, k, x, path=3)
    want = oracle.decode_matrix(raw, Q5K, n, k, dtype=oracle.DTYPE_BF16).T[(7 * np.arange(m)) % k]
    assert np.array_equal(canonical(y), canonical(want))


@pytest.mark.parametrize("m,n,k", [(2, 1000, 768), (8, 3072, 3072), (9, 300, 2048), (33, 3584, 3584),
                                   (64, 18944, 3584), (50, 250, 4096)])
def test_q5k_skinny_matches_oracle(ql, m, n, k):
    path = 3 if m <= 8 else 0  # 2..8 rows run the 2..8-row GEMV unless the skinny kernel is forced
    st, info, _ = plan(Q5K, n, k, m, path=path)
    assert st == 0 and info.kernel == SKINNY
    raw = q5k(n, k, 50 + m)
    x = activations(m, k, 51 + m)
    bias = (np.random.default_rng(52).standard_normal(n) * 0.1).astype(np.float32)
    print(f"[q5k skinny] m={m} n={n} k={k} split={info.workspace_bytes > 0}", flush=True)
    y = run_linear(ql, raw, Q5K, n, k, x, bias=bias, path=path)
    check(f"q5k skinny m={m}", y, *expect(x, decoded(raw, n, k), bias))
    # Deterministic: a second call returns the same bits.
    assert np.array_equal(run_linear(ql, raw, Q5K, n, k, x, bias=bias, path=path), y)


@pytest.mark.parametrize("m,n,k", [(2, 300, 768), (5, 3584, 3584), (8, 18944, 3584), (8, 1000, 2304)])
def test_q5k_gemv8_matches_oracle(ql, m, n, k):
    """2..8 rows on the codes-as-MFMA-operand GEMV (exact fp32 weights; ragged N = 300 and
    1000, an odd super-block count at K = 768 and 2304)."""
    st, info, _ = plan(Q5K, n, k, m)
    assert st == 0 and info.kernel == GEMV8
    raw = q5k(n, k, 70 + m)
    x = activations(m, k, 71 + m)
    bias = (np.random.default_rng(72).standard_normal(n) * 0.1).astype(np.float32)
    print(f"[q5k gemv8] m={m} n={n} k={k}", flush=True)
    y = run_linear(ql, raw, Q5K, n, k, x, bias=bias)
    check(f"q5k gemv8 m={m}", y, *expect(x, decoded(raw, n, k, bf16=False), bias), route="exact")


def test_q5k_gemv8_fused_segments(ql):
    n, k, m = 1536, 1024, 6
    raws = [q5k(n, k, 80 + i) for i in range(3)]
    lins = [ql.QuantizedLinear(torch.from_numpy(r).cuda(), Q5K, n, k) for r in raws]
    x = activations(m, k, 83)
    print("[q5k gemv8] forward_many", flush=True)
    ys = ql.forward_many(lins, to_dev_bf16(x))
    torch.cuda.synchronize()
    for i, (y, r) in enumerate(zip(ys, raws)):
        check(f"q5k gemv8 segment {i}", from_dev_bf16(y), *expect(x, decoded(r, n, k, bf16=False)), route="exact")


def test_q5k_skinny_fused_segments_and_activation(ql):
    n, k, m = 3584, 2048, 40
    raws = [q5k(n, k, 60 + i) for i in range(3)]
    lins = [ql.QuantizedLinear(torch.from_numpy(r).cuda(), Q5K, n, k) for r in raws]
    x = activations(m, k, 63)
    print("[q5k skinny] forward_many", flush=True)
    ys = ql.forward_many(lins, to_dev_bf16(x))
    torch.cuda.synchronize()
    for i, (y, r) in enumerate(zip(ys, raws)):
        check(f"q5k skinny segment {i}", from_dev_bf16(y), *expect(x, decoded(r, n, k)))
    W = ql.Weights()
    W.bind_glu("gu", torch.from_numpy(raws[0]).cuda(), torch.from_numpy(raws[1]).cuda(), Q5K, n, k)
    xd = to_dev_bf16(x)
    pre = from_dev_bf16(W._linears["gu"](xd))
    h = from_dev_bf16(W.project_act(xd, "gu", "silu_glu"))
    want = oracle.act_reference(pre, oracle.ACT_SILU_GLU)
    assert np.count_nonzero(h != want) <= oracle.allowed_differing(h.size, 1e-3)
