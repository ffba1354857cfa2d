"""GPU: grouped projections (tc_qlinear_forward_group): two projections of different
activations (the image and text streams of a dual-stream block, which the reference projects
one after the other, flux_transformer.cpp:995-1004) as one persistent dequant-GEMM grid over
the output tiles of both.

Checks, through the C ABI:
* one-hot activations (different weights per problem) give each problem its own bf16-decoded
  weights bit for bit, for 128- and 256-row tiles, unsplit and split K, ragged N and M: a tile
  read from or written to the other problem's buffers, or a slice summed into the wrong one,
  fails this;
* where the group picks the tile height and K split a problem would pick on its own, that
  problem's outputs equal its own forward bit for bit (same tiles, same K order);
* the config-3 pairs (qk, v, out, mlp_up at 1024 + 256 tokens; qk at 4096 + 256) against the
  oracle on sampled rows, with per-problem biases;
* pairs that cannot share a grid (one projection, mixed types or K, M <= 64, different row
  strides) run each projection's own route and equal forward bit for bit;
* repeated calls are bit-identical;
* output activations: GELU after an unsplit grid (activation pass) and in a split one's slice
  reduction, the gated activation on gate_up bindings (n / 2 wide), against the activation of
  the same launch's pre-activation outputs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from parity import check, expect
from test_gpu_configs import dev_bias, dev_weight, dev_x, host_bf16, oracle_weights, sample_rows
from test_gpu_qlinear import canonical, dense_type_payload

pytestmark = pytest.mark.gpu

Q4K, Q5K, Q6K = 12, 13, 14


@pytest.fixture(scope="module")
def mods():
    from turbocider_amd import gguf, qlinear
    return gguf, qlinear


def weight(gguf, typ, n, k, seed):
    """(device blocks, raw bytes): quantized N(0, 0.02) weights, or random Q5_K blocks under
    small finite scales (the device quantizer covers Q4_K and Q6_K)."""
    if typ == Q5K:
        raw = dense_type_payload(Q5K, n, k, np.random.default_rng(seed))
        return torch.from_numpy(raw).cuda(), raw
    return dev_weight(gguf, typ, n, k, seed)


def one_hot(m, k):
    x = torch.zeros((m, k), dtype=torch.bfloat16, device="cuda")
    x[torch.arange(m), torch.arange(m) % k] = 1.0
    return x


# The group's geometry (the one-problem rules on both problems' tiles together): 128-row tiles
# while both M <= 1024 (<= 512 for K > 8192) and the 256-row tiles number < 160, else 256-row
# tiles; K split in min(K / 512, 256 / tiles) slices when the tiles number < 160 and K >= 1024.
@pytest.mark.parametrize("typ,m0,n0,m1,n1,k", [
    (Q4K, 300, 700, 100, 520, 512),     # 128-row tiles, unsplit (2 super-blocks)
    (Q6K, 300, 700, 100, 520, 1024),    # 128-row tiles, 2 K slices
    (Q4K, 1100, 300, 200, 1000, 1024),  # 256-row tiles (M > 1024), 2 K slices
    (Q5K, 1100, 8192, 90, 256, 512),    # 256-row tiles, unsplit
    (Q6K, 1100, 8192, 70, 300, 512),
])
def test_group_one_hot_returns_each_problems_weights(mods, typ, m0, n0, m1, n1, k):
    gguf, ql = mods
    (b0, r0), (b1, r1) = weight(gguf, typ, n0, k, 11), weight(gguf, typ, n1, k, 12)
    l0, l1 = ql.QuantizedLinear(b0, typ, n0, k), ql.QuantizedLinear(b1, typ, n1, k)
    print(f"[group one-hot] type={typ} m=({m0},{m1}) n=({n0},{n1}) k={k}", flush=True)
    (y0, y1), grouped = ql.forward_group([l0, l1], [one_hot(m0, k), one_hot(m1, k)])
    torch.cuda.synchronize()
    assert grouped
    for y, raw, m, n in ((y0, r0, m0, n0), (y1, r1, m1, n1)):
        want = oracle.decode_matrix(raw, typ, n, k, dtype=oracle.DTYPE_BF16).T[np.arange(m) % k]
        assert np.array_equal(canonical(host_bf16(y)), canonical(want))


def test_group_equals_own_forward_where_the_geometry_matches(mods):
    """Image qk (1024 x 6144, 128-row tiles, unsplit alone and in the group with the 256-row
    text stream) is bit-identical to its own forward; so is the image v projection (split in
    two K slices alone and in the group)."""
    gguf, ql = mods
    for typ, n, seed in ((Q4K, 6144, 21), (Q6K, 3072, 23)):
        (b0, _), (b1, _) = dev_weight(gguf, typ, n, 3072, seed), dev_weight(gguf, typ, n, 3072, seed + 1)
        l0 = ql.QuantizedLinear(b0, typ, n, 3072, dev_bias(n, seed + 2))
        l1 = ql.QuantizedLinear(b1, typ, n, 3072, dev_bias(n, seed + 3))
        x0, x1 = dev_x(1024, 3072, seed + 4), dev_x(256, 3072, seed + 5)
        print(f"[group vs own] type={typ} n={n}", flush=True)
        (g0, g1), grouped = ql.forward_group([l0, l1], [x0, x1])
        own0 = l0(x0)
        torch.cuda.synchronize()
        assert grouped
        assert torch.equal(g0.view(torch.int16), own0.view(torch.int16))
        # Repeated calls: bit-identical (a fixed slice order).
        (h0, h1), _ = ql.forward_group([l0, l1], [x0, x1])
        torch.cuda.synchronize()
        assert torch.equal(h0.view(torch.int16), g0.view(torch.int16))
        assert torch.equal(h1.view(torch.int16), g1.view(torch.int16))


# Config 3 (Qwen-Image-style MMDiT, hidden 3072, MLP 12288): the projections of the image and
# text streams that share type and K.
CONFIG3_PAIRS = [("qk", Q4K, 6144, 3072), ("v", Q6K, 3072, 3072), ("out", Q4K, 3072, 3072),
                 ("mlp_up", Q4K, 12288, 3072)]


@pytest.mark.parametrize("n_img", [1024, 4096])
def test_config3_stream_pairs_match_oracle(mods, n_img):
    gguf, ql = mods
    pairs = CONFIG3_PAIRS if n_img == 1024 else CONFIG3_PAIRS[:1]
    for i, (name, typ, n, k) in enumerate(pairs):
        (b0, r0), (b1, r1) = dev_weight(gguf, typ, n, k, 300 + 2 * i), dev_weight(gguf, typ, n, k, 301 + 2 * i)
        bias0, bias1 = dev_bias(n, 400 + i), dev_bias(n, 500 + i)
        l0, l1 = ql.QuantizedLinear(b0, typ, n, k, bias0), ql.QuantizedLinear(b1, typ, n, k, bias1)
        x0, x1 = dev_x(n_img, k, 600 + i), dev_x(256, k, 700 + i)
        print(f"[config3 group {name}] img={n_img} txt=256 n={n} k={k}", flush=True)
        (y0, y1), grouped = ql.forward_group([l0, l1], [x0, x1])
        torch.cuda.synchronize()
        assert grouped
        for tag, y, x, raw, bias, m, seed in (("img", y0, x0, r0, bias0, n_img, 1), ("txt", y1, x1, r1, bias1, 256, 2)):
            rows = sample_rows(m, seed)
            idx = torch.from_numpy(rows).cuda()
            check(f"config3 {name} {tag} m={m}", host_bf16(y[idx]),
                  *expect(host_bf16(x[idx]), oracle_weights(raw, typ, n, k, m), bias.cpu().numpy()))


def test_pairs_that_do_not_group_run_their_own_routes(mods):
    gguf, ql = mods
    (bq4, _), (bq6, _) = dev_weight(gguf, Q4K, 512, 1024, 31), dev_weight(gguf, Q6K, 512, 1024, 32)
    (bk2, _) = dev_weight(gguf, Q4K, 512, 2048, 33)
    l4, l6 = ql.QuantizedLinear(bq4, Q4K, 512, 1024), ql.QuantizedLinear(bq6, Q6K, 512, 1024)
    l4b, lk2 = ql.QuantizedLinear(bq4, Q4K, 512, 1024), ql.QuantizedLinear(bk2, Q4K, 512, 2048)
    xa, xb = dev_x(300, 1024, 34), dev_x(200, 1024, 35)
    wide = dev_x(200, 1536, 36)[:, :1024]  # row stride 1536, not 1024
    cases = [
        ("one projection", [l4], [xa]),
        ("mixed types", [l4, l6], [xa, xb]),
        ("mixed k", [l4, lk2], [xa, dev_x(200, 2048, 37)]),
        ("64 rows", [l4, l4b], [xa, dev_x(64, 1024, 38)]),
        ("row strides differ", [l4, l4b], [xa, wide]),
    ]
    for name, lins, xs in cases:
        print(f"[group fallback] {name}", flush=True)
        ys, grouped = ql.forward_group(lins, xs)
        torch.cuda.synchronize()
        assert not grouped, name
        for lin, x, y in zip(lins, xs, ys):
            own = lin(x)
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int16), own.view(torch.int16)), name


def test_group_argument_errors(mods):
    gguf, ql = mods
    (b, _) = dev_weight(gguf, Q4K, 256, 512, 41)
    lin = ql.QuantizedLinear(b, Q4K, 256, 512)
    x = dev_x(100, 512, 42)
    with pytest.raises(ql.QLinearError, match="a group holds 1 or 2 projections"):
        ql.forward_group([lin, lin, lin], [x, x, x])
    with pytest.raises(ql.QLinearError, match="one activation per projection"):
        ql.forward_group([lin, lin], [x])
    with pytest.raises(ql.QLinearError, match="last dimension 512"):
        ql.forward_group([lin, lin], [x, dev_x(100, 1024, 43)])


def test_weights_project_group(mods):
    """Weights.project_group: the stream pair through one grouped launch, and a gate_up binding
    with interleaved rows through project() (its output columns are reordered)."""
    gguf, ql = mods
    (b0, _), (b1, _) = dev_weight(gguf, Q4K, 1024, 512, 51), dev_weight(gguf, Q4K, 1024, 512, 52)
    W = ql.Weights()
    W.bind("img.out", b0, Q4K, 1024, 512)
    W.bind("txt.out", b1, Q4K, 1024, 512)
    W.bind_glu("img.gu", b0, b1, Q4K, 1024, 512)
    x0, x1 = dev_x(300, 512, 53), dev_x(100, 512, 54)
    print("[group weights]", flush=True)
    y0, y1 = W.project_group([(x0, "img.out"), (x1, "txt.out")])
    a0, a1 = W.project(x0, "img.out"), W.project(x1, "txt.out")
    g = W.project_group([(x0, "img.gu"), (x1, "txt.out")])
    ga = W.project(x0, "img.gu")
    torch.cuda.synchronize()
    for got, want in ((y0, a0), (g[0], ga), (g[1], a1)):
        assert got.shape == want.shape
    # The grouped pair is checked against the oracle above; here the routing: the gate_up
    # member went through project(), bit-identical.
    assert torch.equal(g[0].view(torch.int16), ga.view(torch.int16))
    with pytest.raises(ql.QLinearError, match="missing weight"):
        W.project_group([(x0, "nothing")])


def test_weights_project_group_with_runtime_lora(mods):
    """A member with a runtime adapter bound routes the pair through project(): both outputs
    equal their own project() bit for bit, and the adapter changes the member's output."""
    gguf, ql = mods
    n, k = 1024, 512
    (b0, _), (b1, _) = dev_weight(gguf, Q4K, n, k, 61), dev_weight(gguf, Q4K, n, k, 62)
    W = ql.Weights()
    W.bind("img.q", b0, Q4K, n, k)
    W.bind("txt.q", b1, Q4K, n, k)
    x0, x1 = dev_x(300, k, 63), dev_x(100, k, 64)
    plain = W.project_group([(x0, "img.q"), (x1, "txt.q")])
    g = torch.Generator(device="cuda").manual_seed(65)
    down = (torch.randn((16, k), generator=g, device="cuda") / 4).to(torch.bfloat16)
    up = (torch.randn((n, 16), generator=g, device="cuda") * 0.01).to(torch.bfloat16)
    W.bind_runtime_lora("txt.q", down, up, 0.8, 16.0)
    print("[group weights lora]", flush=True)
    y0, y1 = W.project_group([(x0, "img.q"), (x1, "txt.q")])
    a0, a1 = W.project(x0, "img.q"), W.project(x1, "txt.q")
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int16), a0.view(torch.int16))
    assert torch.equal(y1.view(torch.int16), a1.view(torch.int16))
    assert not torch.equal(y1.view(torch.int16), plain[1].view(torch.int16))


@pytest.mark.parametrize("n,splits", [(6144, False), (3072, True)])
def test_grouped_gelu(mods, n, splits):
    """GELU on a grouped pair: the activation pass after an unsplit grid (qk-like, 240 tiles) or
    the slice reduction of a split one (v-like, 2 K slices); against the activation of the
    same grouped launch's pre-activation outputs (oracle.act_reference: at most one ulp in
    0.1 % of the outputs)."""
    gguf, ql = mods
    k = 3072
    (b0, _), (b1, _) = dev_weight(gguf, Q4K, n, k, 81), dev_weight(gguf, Q4K, n, k, 82)
    l0 = ql.QuantizedLinear(b0, Q4K, n, k, dev_bias(n, 83))
    l1 = ql.QuantizedLinear(b1, Q4K, n, k, dev_bias(n, 84))
    x0, x1 = dev_x(1024, k, 85), dev_x(256, k, 86)
    print(f"[group gelu] n={n}", flush=True)
    pre, g0 = ql.forward_group([l0, l1], [x0, x1])
    out, g1 = ql.forward_group([l0, l1], [x0, x1], act="gelu_tanh")
    torch.cuda.synchronize()
    assert g0 and g1
    for p, o in zip(pre, out):
        want = oracle.act_reference(host_bf16(p), oracle.ACT_GELU_TANH)
        got = host_bf16(o)
        assert np.count_nonzero(got != want) <= oracle.allowed_differing(got.size, 1e-3)


@pytest.mark.parametrize("n", [6144, 3072])
def test_grouped_silu_glu_on_gate_up_bindings(mods, n):
    """The gated activation on two gate_up bindings (interleaved rows) through project_group:
    n / 2 wide outputs, against the activation of the grouped pre-activation outputs."""
    gguf, ql = mods
    k = 3072
    W = ql.Weights()
    for s, seed in (("img", 91), ("txt", 93)):
        (bg, _), (bu, _) = dev_weight(gguf, Q4K, n // 2, k, seed), dev_weight(gguf, Q4K, n // 2, k, seed + 1)
        W.bind_glu(f"{s}.gu", bg, bu, Q4K, n // 2, k)
    x0, x1 = dev_x(1024, k, 95), dev_x(256, k, 96)
    print(f"[group silu_glu] n={n}", flush=True)
    h0, h1 = W.project_group([(x0, "img.gu"), (x1, "txt.gu")], act="silu_glu")
    pre, grouped = ql.forward_group([W._linears["img.gu"], W._linears["txt.gu"]], [x0, x1])
    torch.cuda.synchronize()
    assert grouped and h0.shape == (1024, n // 2) and h1.shape == (256, n // 2)
    for p, h in zip(pre, (h0, h1)):
        want = oracle.act_reference(host_bf16(p), oracle.ACT_SILU_GLU)
        got = host_bf16(h)
        assert np.count_nonzero(got != want) <= oracle.allowed_differing(got.size, 1e-3)
    with pytest.raises(ql.QLinearError, match="gate_up binding"):
        W.project_group([(x0, "img.gu")], act="gelu_tanh")


def test_activation_on_pairs_that_do_not_group(mods):
    """Mixed types: each member runs tc_qlinear_forward_act, bit-identical to its own call."""
    gguf, ql = mods
    (b4, _), (b6, _) = dev_weight(gguf, Q4K, 1024, 1024, 101), dev_weight(gguf, Q6K, 1024, 1024, 102)
    l4, l6 = ql.QuantizedLinear(b4, Q4K, 1024, 1024), ql.QuantizedLinear(b6, Q6K, 1024, 1024)
    x0, x1 = dev_x(300, 1024, 103), dev_x(200, 1024, 104)
    print("[group act fallback]", flush=True)
    (y0, y1), grouped = ql.forward_group([l4, l6], [x0, x1], act="gelu_tanh")
    a0, a1 = l4.forward(x0, act="gelu_tanh"), l6.forward(x1, act="gelu_tanh")
    torch.cuda.synchronize()
    assert not grouped
    assert torch.equal(y0.view(torch.int16), a0.view(torch.int16))
    assert torch.equal(y1.view(torch.int16), a1.view(torch.int16))
