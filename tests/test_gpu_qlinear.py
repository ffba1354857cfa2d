"""GPU: quantized linear parity (MFMA dequant-GEMM, skinny GEMV, runtime LoRA, bias).

Oracles (oracle/oracle.py):
* GEMM path (bf16 MFMA on bf16-decoded weights): the reference's bf16 decode route
  (decode_cpu_into to bf16, gguf_weight_pager.cpp:347-349) + a float64 GEMM rounded to
  fp32 then bf16; also checked against the fp32-decoded weights for rel-L2.
* GEMV path (exact fp32 weights): CPU dequant to fp32 + GEMM.
* LoRA / bias: the reference sequence pinned by the native_lora_math KATs.
Tolerance (north star): rel-L2 <= 1e-2 and max-abs <= 2e-2 on bf16 outputs, where an output
whose bf16 ulp exceeds 2e-2 (|y| >= 4) may differ by one ulp (one rounding flip).
Exact checks: with one-hot activations the GEMM must return the bf16-decoded weights
bit for bit (size-independent property, also run at the full north-star shape).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from parity import check, check_lora, expect

pytestmark = pytest.mark.gpu

Q4K, Q6K = 12, 14


@pytest.fixture(scope="module")
def ql():
    from turbocider_amd import qlinear
    return qlinear


def weights(typ, n, k, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    return oracle.quantize(typ, w)


def activations(m, k, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return oracle.bf16_bits((rng.standard_normal((m, k)) * scale).astype(np.float32))


def to_dev_bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)


def from_dev_bf16(t: torch.Tensor) -> np.ndarray:
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def run_linear(ql, blocks, typ, n, k, x, bias=None, path=0, adapters=()):
    lin = ql.QuantizedLinear(torch.from_numpy(blocks).cuda(), typ, n, k,
                             torch.from_numpy(bias).cuda() if bias is not None else None)
    lin.set_path(path)
    y = lin(to_dev_bf16(x), adapters)
    torch.cuda.synchronize()
    return from_dev_bf16(y)


def canonical(a: np.ndarray) -> np.ndarray:
    a = a.copy()
    a[(a & 0x7FFF) == 0] = 0
    return a


@pytest.mark.parametrize("typ", [Q4K, Q6K])
def test_gemm_one_hot_returns_bf16_weights_exactly(ql, typ):
    n, k = 300, 512  # N tail (300 = 256 + 44), two super-blocks
    blocks = weights(typ, n, k, 1)
    x = np.zeros((k, k), dtype=np.uint16)
    x[np.arange(k), np.arange(k)] = 0x3F80
    print(f"[one-hot] type={typ}", flush=True)
    y = run_linear(ql, blocks, typ, n, k, x, path=1)
    want = oracle.decode_matrix(blocks, typ, n, k, dtype=oracle.DTYPE_BF16).T
    assert np.array_equal(canonical(y), canonical(want))


@pytest.mark.parametrize("typ", [Q4K, Q6K])
@pytest.mark.parametrize("m,n,k", [(300, 288, 512), (257, 512, 1024), (64, 256, 256)])
def test_gemm_matches_oracle(ql, typ, m, n, k):
    blocks = weights(typ, n, k, 10 + m)
    x = activations(m, k, 20 + m)
    bias = (np.random.default_rng(3).standard_normal(n) * 0.01).astype(np.float32)
    y = run_linear(ql, blocks, typ, n, k, x, bias=bias, path=1)
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, typ, n, k, dtype=oracle.DTYPE_BF16))
    check(f"gemm t{typ} {m}x{n}x{k}", y, *expect(x, wb, bias))
    wf = oracle.decode_matrix(blocks, typ, n, k)
    assert oracle.compare_bf16(y, oracle.linear_reference(x, wf, oracle.bias_to_bf16(bias)))["rel_l2"] < 1e-2


@pytest.mark.parametrize("typ,m,n,k", [
    (Q4K, 4352, 4096, 256),   # 272 single-super-block items: more items than CUs, every
                              # item is its own last block (stream hand-over at each item)
    (Q6K, 4100, 4352, 512),   # 17 x 17 tiles, ragged last M tile: edge tiles between full ones
])
def test_gemm_persistent_stream_matches_oracle(ql, typ, m, n, k):
    """Persistent workgroups walk several output tiles as one K stream (prefetching the next
    tile's first chunks, overlapping the epilogue stores): check every output."""
    blocks = weights(typ, n, k, 110 + m)
    x = activations(m, k, 111)
    bias = (np.random.default_rng(112).standard_normal(n) * 0.01).astype(np.float32)
    print(f"[persistent] type={typ} {m}x{n}x{k}", flush=True)
    y = run_linear(ql, blocks, typ, n, k, x, bias=bias, path=1)
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, typ, n, k, dtype=oracle.DTYPE_BF16))
    check(f"persistent t{typ} {m}x{n}x{k}", y, *expect(x, wb, bias))


@pytest.mark.parametrize("typ,m,n,k", [
    (Q4K, 1, 300, 768),       # 32-row tile, K split (2 tiles, 3 slices), N tail
    (Q6K, 7, 300, 768),
    (Q4K, 32, 520, 1024),     # full 32-row tile
    (Q6K, 33, 300, 1280),     # 64-row tile, one row into the second block
    (Q4K, 64, 257, 512),
    (Q6K, 20, 81920, 256),    # 32-row tile, 320 tiles: no split, persistent (two per CU)
    (Q4K, 40, 81920, 256),    # 64-row tile, no split
])
def test_gemm_skinny_tiles_match_oracle(ql, typ, m, n, k):
    """Small M runs the GEMM with 32- or 64-row tiles (fewer MFMAs per weight; the dequant is
    shared the same way): split and unsplit grids, ragged M and N."""
    blocks = weights(typ, n, k, 80 + m)
    x = activations(m, k, 81 + m)
    bias = (np.random.default_rng(82).standard_normal(n) * 0.01).astype(np.float32)
    print(f"[skinny] type={typ} {m}x{n}x{k}", flush=True)
    y = run_linear(ql, blocks, typ, n, k, x, bias=bias, path=1)
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, typ, n, k, dtype=oracle.DTYPE_BF16))
    check(f"skinny t{typ} {m}x{n}x{k}", y, *expect(x, wb, bias))


@pytest.mark.parametrize("typ,m,n,k", [
    (Q4K, 9, 300, 768),        # one 16-row group, 5 tiles, 3 super-blocks (no split)
    (Q6K, 16, 64, 2048),       # one tile, K split 4 ways (two super-blocks each)
    (Q4K, 17, 3584, 3584),     # text-encoder q/k/v/o: 2 row groups, K split 4 ways
    (Q6K, 32, 200, 256),       # single super-block, ragged last tile
    (Q4K, 33, 18944, 3584),    # text-encoder gate/up: 296 tiles, no split
    (Q6K, 64, 3584, 18944),    # text-encoder down: K split 4 ways (18 or 19 blocks per slice)
    (Q4K, 64, 11000, 512),     # 172 tiles, no split, ragged N
    (Q6K, 47, 12288, 1280),    # 5 super-blocks per slice (prefetch clamped at the slice end)
    (Q4K, 20, 250, 2048),      # K split 4 ways with N % 4 == 2 (the slice sum's element path)
])
def test_skinny_mid_m_matches_oracle(ql, typ, m, n, k):
    """9..64 rows: activations shared through LDS per 64-row weight tile, weights decoded once
    to bf16 (the GEMM's bf16-decode route), optional K split summed in slice order; checked
    with and without a bias, and against the MFMA GEMM forced on the same inputs."""
    blocks = weights(typ, n, k, 130 + m)
    x = activations(m, k, 131 + m)
    bias = (np.random.default_rng(132).standard_normal(n) * 0.01).astype(np.float32)
    print(f"[skinny-mid] type={typ} {m}x{n}x{k}", flush=True)
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, typ, n, k, dtype=oracle.DTYPE_BF16))
    y = run_linear(ql, blocks, typ, n, k, x, bias=bias)
    check(f"skinny-mid t{typ} {m}x{n}x{k}", y, *expect(x, wb, bias))
    y0 = run_linear(ql, blocks, typ, n, k, x, path=3)
    check(f"skinny-mid nobias t{typ} {m}x{n}x{k}", y0, *expect(x, wb))
    # Deterministic: a second call returns the same bits.
    assert np.array_equal(run_linear(ql, blocks, typ, n, k, x, path=3), y0)


@pytest.mark.parametrize("typ", [Q4K, Q6K])
@pytest.mark.parametrize("m", [1, 4, 8])
def test_skinny_forced_small_m_matches_oracle(ql, typ, m):
    """The skinny kernel forced at 1..8 rows (rows past M read zero through the buffer range
    check and are never stored)."""
    n, k = 520, 1536
    blocks = weights(typ, n, k, 140 + m)
    x = activations(m, k, 141 + m)
    y = run_linear(ql, blocks, typ, n, k, x, path=3)
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, typ, n, k, dtype=oracle.DTYPE_BF16))
    check(f"skinny-forced t{typ} m={m}", y, *expect(x, wb))


@pytest.mark.parametrize("typ", [Q4K, Q6K])
@pytest.mark.parametrize("m,n,k", [(2, 300, 256), (3, 300, 768), (5, 1000, 3584), (8, 3584, 3584),
                                   (8, 37, 512), (4, 16, 18944), (7, 200, 1280)])
def test_gemv8_small_m_matches_oracle(ql, typ, m, n, k):
    """2..8 rows (one MFMA per 32-weight step over all rows, scales on the outputs; Q6_K with
    its two 16-weight scale groups per step): exact fp32 weights, so the oracle is the
    fp32-decode GEMM; an odd super-block count (a Q4_K half set), ragged N, a single tile,
    long K."""
    blocks = weights(typ, n, k, 120 + m)
    x = activations(m, k, 121 + m)
    bias = (np.random.default_rng(122).standard_normal(n) * 0.01).astype(np.float32)
    print(f"[gemv8] type={typ} {m}x{n}x{k}", flush=True)
    y = run_linear(ql, blocks, typ, n, k, x, bias=bias)
    wf = oracle.decode_matrix(blocks, typ, n, k)
    check(f"gemv8 t{typ} {m}x{n}x{k}", y, *expect(x, wf, bias), route="exact")


@pytest.mark.parametrize("typ", [Q4K, Q6K])
@pytest.mark.parametrize("m", [1, 3, 8, 12])
def test_forward_many_matches_oracle(ql, typ, m):
    """Projections of one activation (q/k/v-like, one with a bias): one fused launch for
    m <= 8 (the one-row or the 2..8-row kernel over all weights, exact fp32 weights),
    separate GEMM launches otherwise (bf16-decode route); each output matches its own
    projection's oracle."""
    k = 768
    ns = (384, 128, 200)
    rng = np.random.default_rng(95)
    x = activations(m, k, 96)
    blocks = [weights(typ, n, k, 97 + i) for i, n in enumerate(ns)]
    biases = [None, (rng.standard_normal(128) * 0.01).astype(np.float32), None]
    lins = [ql.QuantizedLinear(torch.from_numpy(b).cuda(), typ, n, k,
                               torch.from_numpy(bb).cuda() if bb is not None else None)
            for b, n, bb in zip(blocks, ns, biases)]
    print(f"[many] type={typ} m={m}", flush=True)
    ys = ql.forward_many(lins, to_dev_bf16(x))
    torch.cuda.synchronize()
    for y, b, n, bb in zip(ys, blocks, ns, biases):
        got = from_dev_bf16(y)
        w = oracle.decode_matrix(b, typ, n, k)
        if m > 8:
            w = oracle.bf16_to_f32(oracle.decode_matrix(b, typ, n, k, dtype=oracle.DTYPE_BF16))
        check(f"many t{typ} m={m} n={n}", got, *expect(x, w, bb), route="exact" if m <= 8 else "bf16")


@pytest.mark.parametrize("typ", [Q4K, Q6K])
@pytest.mark.parametrize("m", [20, 64])
def test_forward_many_skinny_fused_matches_oracle(ql, typ, m):
    """9..64 rows, projections of one activation holding >= 128 tiles of 64 rows: one fused
    skinny launch over the three weights (K unsplit; ragged last tile, one bias), each output
    against its own bf16-decode oracle."""
    k = 1024
    ns = (4096, 2048, 2200)
    rng = np.random.default_rng(180)
    x = activations(m, k, 181)
    blocks = [weights(typ, n, k, 182 + i) for i, n in enumerate(ns)]
    biases = [None, (rng.standard_normal(2048) * 0.01).astype(np.float32), None]
    lins = [ql.QuantizedLinear(torch.from_numpy(b).cuda(), typ, n, k,
                               torch.from_numpy(bb).cuda() if bb is not None else None)
            for b, n, bb in zip(blocks, ns, biases)]
    print(f"[many-skinny] type={typ} m={m}", flush=True)
    ys = ql.forward_many(lins, to_dev_bf16(x))
    torch.cuda.synchronize()
    for y, b, n, bb in zip(ys, blocks, ns, biases):
        wb = oracle.bf16_to_f32(oracle.decode_matrix(b, typ, n, k, dtype=oracle.DTYPE_BF16))
        check(f"many-skinny t{typ} m={m} n={n}", from_dev_bf16(y), *expect(x, wb, bb))


@pytest.mark.parametrize("typ", [Q4K, Q6K])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8])
def test_gemv_matches_oracle(ql, typ, m):
    n, k = 300, 768
    blocks = weights(typ, n, k, 30 + m)
    x = activations(m, k, 40 + m)
    bias = (np.random.default_rng(4).standard_normal(n) * 0.01).astype(np.float32)
    y = run_linear(ql, blocks, typ, n, k, x, bias=bias, path=2)
    wf = oracle.decode_matrix(blocks, typ, n, k)
    check(f"gemv t{typ} m={m}", y, *expect(x, wf, bias), route="exact")


@pytest.mark.parametrize("typ,m,n,k", [
    (Q4K, 200, 20480, 512),   # 128-row tiles (few 256-row tiles): 2 x 80 tiles, no split
    (Q6K, 330, 10240, 512),   # 128-row tiles, ragged last M tile, no split (2 super-blocks)
])
def test_gemm_128_row_tiles_match_oracle(ql, typ, m, n, k):
    """65..512 rows whose 256-row tiling leaves the grid short of tiles run 128-row tiles."""
    blocks = weights(typ, n, k, 160 + m)
    x = activations(m, k, 161)
    bias = (np.random.default_rng(162).standard_normal(n) * 0.01).astype(np.float32)
    print(f"[gemm-128] type={typ} {m}x{n}x{k}", flush=True)
    y = run_linear(ql, blocks, typ, n, k, x, bias=bias, path=1)
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, typ, n, k, dtype=oracle.DTYPE_BF16))
    check(f"gemm-128 t{typ} {m}x{n}x{k}", y, *expect(x, wb, bias))


@pytest.mark.parametrize("typ,m,n,k", [
    (Q4K, 4132, 4096, 512),   # LTX token count: 16 x 16 full 256-row tiles (one grid round) + 36 rows
    (Q6K, 2600, 6400, 512),   # 10 x 25 full tiles (one round) + 40 rows
])
def test_gemm_tail_rows_on_skinny_kernel(ql, typ, m, n, k):
    """A short last row of 256-row tiles that would cost a grid round of its own runs on the
    skinny kernel after the GEMM (bf16-decode route on both): every row, with a bias."""
    blocks = weights(typ, n, k, 170 + m)
    x = activations(m, k, 171)
    bias = (np.random.default_rng(172).standard_normal(n) * 0.01).astype(np.float32)
    print(f"[gemm-tail] type={typ} {m}x{n}x{k}", flush=True)
    y = run_linear(ql, blocks, typ, n, k, x, bias=bias)
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, typ, n, k, dtype=oracle.DTYPE_BF16))
    want, chain, S = expect(x, wb, bias)
    check(f"gemm-tail t{typ} {m}x{n}x{k}", y, want, chain, S)
    tail = m % 256
    check(f"gemm-tail rows t{typ}", y[-tail:], want[-tail:], [c[-tail:] for c in chain], S[-tail:])


@pytest.mark.parametrize("typ,m,n,k", [
    (Q6K, 64, 3584, 18944),   # text-encoder down at M=64: 14 tiles, K split 16 ways
    (Q4K, 200, 1000, 7168),   # 4 tiles, K split 14 ways, N tail
    (Q4K, 300, 300, 2048),    # ragged M and N tiles, K split 4 ways
])
def test_gemm_split_k_matches_oracle(ql, typ, m, n, k):
    """Grids with few output tiles split K across workgroups; the fp32 slices are summed in
    a fixed order by a second kernel (then bf16, then the bias)."""
    blocks = weights(typ, n, k, 70 + m)
    x = activations(m, k, 71)
    bias = (np.random.default_rng(72).standard_normal(n) * 0.01).astype(np.float32)
    print(f"[split-k] type={typ} {m}x{n}x{k}", flush=True)
    y = run_linear(ql, blocks, typ, n, k, x, bias=bias, path=1)
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, typ, n, k, dtype=oracle.DTYPE_BF16))
    check(f"split-k t{typ} {m}x{n}x{k}", y, *expect(x, wb, bias))


@pytest.mark.parametrize("typ,n,k", [
    (Q4K, 18944, 3584),  # text-encoder gate/up: two 16-row tiles per workgroup
    (Q6K, 3584, 18944),  # text-encoder down: three sets per wavefront, two passes over K
    (Q4K, 40, 2304),     # odd number of super-blocks: the last two-block set is half empty
    (Q4K, 17, 16896),    # 33 sets: three per wavefront, ragged last wavefront
    (Q6K, 33, 256),      # a single set, row tail
])
def test_gemv_single_row_matches_oracle(ql, typ, n, k):
    """M = 1 (block-diagonal MFMA path) at the text-encoder shapes and at the edge shapes of
    its work split, against the fp32-dequant GEMV."""
    blocks = weights(typ, n, k, 60 + n % 7)
    x = activations(1, k, 61)
    bias = (np.random.default_rng(62).standard_normal(n) * 0.01).astype(np.float32)
    wf = oracle.decode_matrix(blocks, typ, n, k)
    for b in (bias, None):
        print(f"[gemv m=1] type={typ} n={n} k={k} bias={b is not None}", flush=True)
        y = run_linear(ql, blocks, typ, n, k, x, bias=b, path=2)
        check(f"gemv1 t{typ} {n}x{k}", y, *expect(x, wf, b), route="exact")
    # Tiles shared by several wavefronts are summed in a fixed order through the handle's
    # workspace, whose counters each call re-arms: repeated calls are bit-identical.
    lin = ql.QuantizedLinear(torch.from_numpy(blocks).cuda(), typ, n, k, torch.from_numpy(bias).cuda())
    lin.set_path(2)
    xd = to_dev_bf16(x)
    outs = [from_dev_bf16(lin(xd)) for _ in range(3)]
    torch.cuda.synchronize()
    assert all(np.array_equal(outs[0], o) for o in outs[1:])
    check(f"gemv1 t{typ} {n}x{k} repeated", outs[2], *expect(x, wf, bias), route="exact")


def test_config1_q4k_linear_full_size(ql):
    """W[3072,3072] N(0,0.02) seed 0, X[1024,3072] N(0,1), bias N(0,0.01)."""
    n = k = 3072
    m = 1024
    blocks = weights(Q4K, n, k, 0)
    x = activations(m, k, 1)
    bias = (np.random.default_rng(2).standard_normal(n) * 0.01).astype(np.float32)
    y = run_linear(ql, blocks, Q4K, n, k, x, bias=bias)
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, Q4K, n, k, dtype=oracle.DTYPE_BF16))
    check("config1 vs bf16-decoded", y, *expect(x, wb, bias))
    wf = oracle.decode_matrix(blocks, Q4K, n, k)
    stats = oracle.compare_bf16(y, oracle.linear_reference(x, wf, oracle.bias_to_bf16(bias)))
    print(f"[config1 vs fp32-decoded] {stats}", flush=True)
    assert stats["rel_l2"] < 1e-2


def test_runtime_lora_segments_and_fused_ranges(ql):
    """Config-5 style: 4 images, each with its own adapter (r in {16, 64, 20, 64}); one adapter
    targets a fused output range; a second adapter stacks on image 0; bias last."""
    n, k, per = 384, 512, 96
    m = 4 * per
    blocks = weights(Q4K, n, k, 50)
    x = activations(m, k, 51)
    bias = (np.random.default_rng(52).standard_normal(n) * 0.01).astype(np.float32)
    rng = np.random.default_rng(53)
    specs = [(0, 16, 0, n), (1, 64, 0, n), (2, 20, 128, 320), (3, 64, 0, n), (0, 64, 0, n)]
    adapters, oracle_ads = [], []
    for img, r, ob, oe in specs:
        a = oracle.bf16_bits((rng.standard_normal((r, k)) / np.sqrt(r)).astype(np.float32))
        b = oracle.bf16_bits((rng.standard_normal((oe - ob, r)) * 0.01).astype(np.float32))
        s = float(np.float32(rng.uniform(0.5, 1.5)))
        adapters.append(ql.LoRAAdapter(to_dev_bf16(a), to_dev_bf16(b), s, img * per, per, ob, oe))
        oracle_ads.append(dict(a=a, b=b, scale=s, row_begin=img * per, row_count=per, out_begin=ob, out_end=oe))
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, Q4K, n, k, dtype=oracle.DTYPE_BF16))
    for path in (1, 0):
        print(f"[lora] path={path}", flush=True)
        y = run_linear(ql, blocks, Q4K, n, k, x, bias=bias, path=path, adapters=adapters)
        base = run_linear(ql, blocks, Q4K, n, k, x, path=path)
        check_lora(f"lora path={path}", y, base, x, wb, bias, oracle_ads)


@pytest.mark.parametrize("typ", [Q4K, Q6K])
def test_runtime_lora_on_skinny_rows(ql, typ):
    """9..64 rows with runtime adapters (the text-encoder prompt route): the skinny kernel's
    output (split and unsplit K), then the adapters in order and the bias last."""
    m, k = 40, 2048
    x = activations(m, k, 151)
    rng = np.random.default_rng(152)
    for n in (256, 12288):   # 4 tiles: K split 2 ways; 192 tiles: no split
        blocks = weights(typ, n, k, 150 + n)
        bias = (rng.standard_normal(n) * 0.01).astype(np.float32)
        specs = [(0, 24, 16, 0, n), (8, 32, 64, n // 4, n // 2)]
        adapters, oracle_ads = [], []
        for rb, rc, r, ob, oe in specs:
            a = oracle.bf16_bits((rng.standard_normal((r, k)) / np.sqrt(r)).astype(np.float32))
            b = oracle.bf16_bits((rng.standard_normal((oe - ob, r)) * 0.01).astype(np.float32))
            sc = float(np.float32(rng.uniform(0.5, 1.5)))
            adapters.append(ql.LoRAAdapter(to_dev_bf16(a), to_dev_bf16(b), sc, rb, rc, ob, oe))
            oracle_ads.append(dict(a=a, b=b, scale=sc, row_begin=rb, row_count=rc, out_begin=ob, out_end=oe))
        print(f"[lora-skinny] type={typ} {m}x{n}x{k}", flush=True)
        y = run_linear(ql, blocks, typ, n, k, x, bias=bias, adapters=adapters)
        base = run_linear(ql, blocks, typ, n, k, x)
        wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, typ, n, k, dtype=oracle.DTYPE_BF16))
        check_lora(f"lora-skinny t{typ} n={n}", y, base, x, wb, bias, oracle_ads)


def test_runtime_lora_many_adapters_ragged(ql):
    """More adapters than one kernel batch (11: applied in two passes, in order), overlapping
    row ranges, ragged M / N (tiles cut by the edges), odd ranks, partial output ranges."""
    n, k, m = 200, 256, 100
    blocks = weights(Q4K, n, k, 60)
    x = activations(m, k, 61)
    bias = (np.random.default_rng(62).standard_normal(n) * 0.01).astype(np.float32)
    rng = np.random.default_rng(63)
    adapters, oracle_ads = [], []
    for i in range(11):
        r = int(rng.choice([1, 7, 16, 33]))
        rb = int(rng.integers(0, m - 1))
        rc = int(rng.integers(1, m - rb + 1))
        ob = int(rng.integers(0, n - 1))
        oe = int(rng.integers(ob + 1, n + 1))
        a = oracle.bf16_bits((rng.standard_normal((r, k)) / np.sqrt(r)).astype(np.float32))
        b = oracle.bf16_bits((rng.standard_normal((oe - ob, r)) * 0.05).astype(np.float32))
        s = float(np.float32(rng.uniform(-1.5, 1.5)))
        adapters.append(ql.LoRAAdapter(to_dev_bf16(a), to_dev_bf16(b), s, rb, rc, ob, oe))
        oracle_ads.append(dict(a=a, b=b, scale=s, row_begin=rb, row_count=rc, out_begin=ob, out_end=oe))
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, Q4K, n, k, dtype=oracle.DTYPE_BF16))
    for path in (1, 0):
        print(f"[lora many] path={path}", flush=True)
        y = run_linear(ql, blocks, Q4K, n, k, x, bias=bias, path=path, adapters=adapters)
        base = run_linear(ql, blocks, Q4K, n, k, x, path=path)
        check_lora(f"lora many path={path}", y, base, x, wb, bias, oracle_ads)


def test_runtime_lora_kat_through_gpu(ql):
    """native_lora_math_test.cpp:127-151 on the device: base y = -256, low = 1.00390625 kept in
    fp32, B = 256 -> bf16(-256 + 257) = 1 (a bf16-narrowed low would give 0); bias 0 last."""
    k, n = 256, 1
    blk = np.zeros(oracle.BLOCK_BYTES[Q4K], dtype=np.uint8)
    blk[0:2] = np.frombuffer(np.float16(256.0).tobytes(), dtype=np.uint8)  # d
    blk[2:4] = np.frombuffer(np.float16(256.0).tobytes(), dtype=np.uint8)  # dmin
    blk[4] = 1       # sc[0] = 1
    blk[8] = 1       # m[0] = 1
    blk[16 + 1] = 1  # q[1] = 1 -> w[0] = -256, w[1] = 0
    dec = oracle.decode_matrix(blk, Q4K, 1, k)
    assert dec[0, 0] == -256.0 and dec[0, 1] == 0.0
    x = np.zeros((1, k), dtype=np.uint16)
    x[0, :2] = 0x3F80
    a = np.zeros((16, k), dtype=np.uint16)
    a[0, 0], a[0, 1] = 0x3F80, 0x3B80
    b = np.zeros((1, 16), dtype=np.uint16)
    b[0, 0] = 0x4380
    bias = np.zeros(1, dtype=np.float32)
    for path in (1, 2):
        y = run_linear(ql, blk, Q4K, n, k, x, bias=bias, path=path,
                       adapters=[ql.LoRAAdapter(to_dev_bf16(a), to_dev_bf16(b), 1.0)])
        assert y[0, 0] == 0x3F80, (path, hex(y[0, 0]))


def test_northstar_shape_exact_dequant_and_sampled_rows(ql):
    """M=4096, K=3072, N=12288 (the north-star GEMM): one-hot rows give the whole bf16 weight
    matrix bit for bit; random rows match the oracle."""
    from turbocider_amd import gguf
    m, k, n = 4096, 3072, 12288
    rng = torch.Generator(device="cuda").manual_seed(0)
    w = (torch.randn((n, k), generator=rng, device="cuda") * 0.02).contiguous()
    blocks = gguf.quantize(w, Q4K)
    del w
    lin = ql.QuantizedLinear(blocks, Q4K, n, k)
    x = torch.zeros((m, k), dtype=torch.bfloat16, device="cuda")
    x[torch.arange(k), torch.arange(k)] = 1.0
    print("[northstar] one-hot", flush=True)
    y = lin(x)
    wb = gguf.dequantize(blocks, Q4K, n, k, gguf.DecodeDType.bf16)
    got = y[:k].t().contiguous().view(torch.int16)
    want = wb.view(torch.int16)
    zero_g, zero_w = (got & 0x7FFF) == 0, (want & 0x7FFF) == 0
    assert torch.equal(zero_g, zero_w) and torch.equal(got[~zero_g], want[~zero_w])
    assert (y[k:].float() == 0).all()
    print("[northstar] sampled rows", flush=True)
    xr = torch.randn((m, k), generator=rng, device="cuda").to(torch.bfloat16)
    y = lin(xr)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 31, 32, 255, 256, 1000, 2047, 2048, 3333, 4064, 4095])
    wb_np = oracle.bf16_to_f32(from_dev_bf16(wb))
    want = oracle.linear_reference(from_dev_bf16(xr)[rows], wb_np)
    check("northstar rows", from_dev_bf16(y)[rows], want, term_sum=oracle.abs_term_sum(from_dev_bf16(xr)[rows], wb_np))
    # the device decode of the full tensor is bit-exact to the oracle's
    assert np.array_equal(from_dev_bf16(wb), oracle.decode_matrix(blocks.cpu().numpy(), Q4K, n, k,
                                                                    dtype=oracle.DTYPE_BF16))


def dense_type_payload(typ, n, k, rng):
    """Raw rows of a non-Q4_K/Q6_K type whose decoded weights look like N(0, 0.02) weights:
    floats directly, blocks with random codes under small finite scales (and minimums)."""
    bb, el = oracle.BLOCK_BYTES[typ], oracle.BLOCK_ELEMENTS[typ]
    if typ in (0, 1, 30):
        w = (rng.standard_normal(n * k) * 0.02).astype(np.float32)
        return (w if typ == 0 else w.astype(np.float16) if typ == 1 else oracle.bf16_bits(w)).view(np.uint8)
    raw = rng.integers(0, 256, size=n * k // el * bb, dtype=np.uint8)
    blocks = raw.reshape(-1, bb)
    scale = {13: 0.00003, 8: 0.0005, 2: 0.005, 3: 0.005, 6: 0.0025, 7: 0.0025}[typ]
    blocks[:, 0:2] = np.frombuffer(np.float16(scale).tobytes() * len(blocks), dtype=np.uint8).reshape(-1, 2)
    if typ in (13, 3, 7):  # dmin / minimum
        blocks[:, 2:4] = np.frombuffer(np.float16(-0.04 if typ != 13 else 0.00006).tobytes() * len(blocks),
                                       dtype=np.uint8).reshape(-1, 2)
    return raw


@pytest.mark.parametrize("typ", [8, 2, 3, 6, 7, 1, 30, 0])
def test_dense_types_projection_matches_oracle(ql, typ):
    """A projection over each of the other registered types (decoded once to bf16, library GEMM):
    M = 1, 7 and 300 rows with a bias and one runtime adapter, against the oracle's
    decode-to-bf16 + fp32 GEMM reference (the reference's dense branch, mlx.cpp:680-686)."""
    n, k = 300, 512
    rng = np.random.default_rng(200 + typ)
    raw = dense_type_payload(typ, n, k, rng)
    status, dec, _, err = oracle.decode_raw(raw.tobytes(), typ, n, k, dtype=2)
    assert status == 0, err
    wb = oracle.bf16_to_f32(np.frombuffer(dec, dtype=np.uint16).reshape(n, k))
    bias = (rng.standard_normal(n) * 0.01).astype(np.float32)
    r = 16
    a = oracle.bf16_bits((rng.standard_normal((r, k)) / np.sqrt(r)).astype(np.float32))
    b = oracle.bf16_bits((rng.standard_normal((n - 20, r)) * 0.01).astype(np.float32))
    for m in (1, 7, 300):
        x = activations(m, k, 300 + m)
        ads = [dict(a=a, b=b, scale=0.75, row_begin=0, row_count=m, out_begin=10, out_end=n - 10)]
        print(f"[dense] type={typ} m={m}", flush=True)
        y = run_linear(ql, raw, typ, n, k, x, bias=bias,
                       adapters=[ql.LoRAAdapter(to_dev_bf16(a), to_dev_bf16(b), 0.75, 0, m, 10, n - 10)])
        base = run_linear(ql, raw, typ, n, k, x)
        check_lora(f"dense {typ} m={m}", y, base, x, wb, bias, ads)
        y0 = run_linear(ql, raw, typ, n, k, x, bias=bias)
        check(f"dense {typ} m={m} no lora", y0, *expect(x, wb, bias))


def test_dense_type_rejects_nonfinite_weights(ql):
    """Creation decodes the weights and rejects a non-finite value with the reference's message."""
    raw = np.zeros(4 * 256 * 2, dtype=np.uint8)
    raw[2 * 77:2 * 77 + 2] = np.frombuffer(np.uint16(0x7C00).tobytes(), dtype=np.uint8)
    with pytest.raises(ql.QLinearError, match="nonfinite weight/scale or conversion overflow"):
        ql.QuantizedLinear(torch.from_numpy(raw).cuda(), 1, 4, 256)
