"""GPU: parity at every BASELINE configuration's real shapes, through the C ABI.

Weights are N(0, 0.02) fp32 quantized on the device (tc_gguf_quantize_device, bit-identical to
the oracle's quantizer, test_gpu_decode.py); activations N(0, 1) bf16; biases N(0, 0.01). The
oracle decodes the same raw blocks on the CPU (oracle/tc_oracle.c) and runs a float64 GEMM
rounded to fp32 then bf16, on

* every output row where that is cheap (config 2: the text-encoder block at M = 1, 8, 64, 256),
* sampled rows otherwise (every tile edge, the split / tail boundaries, random rows),
  since each output row depends only on its own activation row;

and with one-hot activations the long-K Q6_K projections must return the bf16-decoded weight
matrix bit for bit (a size-independent property of the dequant-GEMM).

Oracle weights follow the kernel's decode route: exact fp32 weights for the 1..8-row GEMVs,
bf16-decoded weights for the skinny kernel and the MFMA GEMM (the reference pager's bf16
decode, gguf_weight_pager.cpp:347-349). Bounds: tests/parity.py (the north-star tolerance and
the tight summation-order bound); runtime LoRA is checked in stages there (base projection,
adapters on the kernel's own base, end to end).
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
def mods():
    from turbocider_amd import gguf, qlinear
    return gguf, qlinear


def dev_weight(gguf, typ, n, k, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn((n, k), generator=g, device="cuda") * 0.02
    blocks = gguf.quantize(w, typ)
    torch.cuda.synchronize()
    return blocks, blocks.cpu().numpy()


def dev_x(m, k, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)


def dev_bias(n, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(n, generator=g, device="cuda") * 0.01


def host_bf16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def sample_rows(m, seed, extra=()):
    """Tile and split edges (multiples of 16 / 32 / 64 / 128 / 256 and their neighbours), the
    last 64 rows (a GEMM tail run by the skinny kernel), and random rows."""
    edges = {0, 1, m - 1}
    for step in (16, 32, 64, 128, 256):
        for b in range(step, m, step * max(1, m // (4 * step))):
            edges.update((b - 1, b))
    edges.update(range(max(0, m - 64), m, 7))
    edges.update(np.random.default_rng(seed).integers(0, m, 24).tolist())
    edges.update(extra)
    return np.array(sorted(r for r in edges if 0 <= r < m))


def oracle_weights(raw, typ, n, k, m):
    """Decoded weights of the route the kernels take at m rows (fp32 exact for m <= 8)."""
    if m <= 8:
        return oracle.decode_matrix(raw, typ, n, k)
    return oracle.bf16_to_f32(oracle.decode_matrix(raw, typ, n, k, dtype=oracle.DTYPE_BF16))


def route(m):
    return "exact" if m <= 8 else "bf16"


def run_projection(mods, name, typ, n, k, m, seed, rows=None, with_bias=True):
    """One projection at its real shape: the kernel's output on `rows` (all when None) vs the
    oracle. Returns (linear, x, y) for further checks."""
    gguf, ql = mods
    blocks, raw = dev_weight(gguf, typ, n, k, seed)
    bias = dev_bias(n, seed + 1) if with_bias else None
    lin = ql.QuantizedLinear(blocks, typ, n, k, bias)
    x = dev_x(m, k, seed + 2)
    print(f"[{name}] type={typ} m={m} n={n} k={k}", flush=True)
    y = lin(x)
    torch.cuda.synchronize()
    idx = np.arange(m) if rows is None else rows
    xh = host_bf16(x[torch.from_numpy(idx).cuda()])
    yh = host_bf16(y[torch.from_numpy(idx).cuda()])
    check(name, yh, *expect(xh, oracle_weights(raw, typ, n, k, m), bias.cpu().numpy() if bias is not None else None),
          route=route(m))
    return lin, x, y


# ---- config 2: text-encoder block (q/k/v/o 3584^2 Q4_K, gate/up 3584 -> 18944 Q4_K, down
# 18944 -> 3584 Q6_K) at M in {1, 8, 64, 256}, every output --------------------------------
CONFIG2 = [("q", Q4K, 3584, 3584), ("k", Q4K, 3584, 3584), ("v", Q4K, 3584, 3584), ("o", Q4K, 3584, 3584),
           ("gate", Q4K, 18944, 3584), ("up", Q4K, 18944, 3584), ("down", Q6K, 3584, 18944)]


@pytest.fixture(scope="module")
def config2(mods):
    gguf, ql = mods
    out = {}
    for i, (name, typ, n, k) in enumerate(CONFIG2):
        blocks, raw = dev_weight(gguf, typ, n, k, 100 + i)
        out[name] = (ql.QuantizedLinear(blocks, typ, n, k), raw, typ, n, k)
    return out


@pytest.mark.parametrize("m", [1, 8, 64, 256])
def test_config2_block_every_output(mods, config2, m):
    for name, (lin, raw, typ, n, k) in config2.items():
        x = dev_x(m, k, 200 + m + (1000 if name == "down" else 0))
        print(f"[config2 {name}] m={m}", flush=True)
        y = lin(x)
        torch.cuda.synchronize()
        check(f"config2 {name} m={m}", host_bf16(y), *expect(host_bf16(x), oracle_weights(raw, typ, n, k, m)),
              route=route(m))


@pytest.mark.parametrize("m", [1, 8, 64, 256])
def test_config2_fused_projections(mods, config2, m):
    """q/k/v and gate/up as projections of one activation (tc_qlinear_forward_many): one
    launch at m <= 64, separate GEMMs at m = 256; every output against its own oracle."""
    _, ql = mods
    x = dev_x(m, 3584, 300 + m)
    xh = host_bf16(x)
    for group in (("q", "k", "v"), ("gate", "up")):
        print(f"[config2 fused {'+'.join(group)}] m={m}", flush=True)
        ys = ql.forward_many([config2[g][0] for g in group], x)
        torch.cuda.synchronize()
        for g, y in zip(group, ys):
            _, raw, typ, n, k = config2[g]
            check(f"config2 fused {g} m={m}", host_bf16(y), *expect(xh, oracle_weights(raw, typ, n, k, m)),
                  route=route(m))


# ---- config 3: Qwen-Image MMDiT block, hidden 3072, MLP 12288 ------------------------------
# Per stream: q, k 3072 -> 6144 (fused qk), v 3072 -> 3072 Q6_K, out 3072 -> 3072, up
# 3072 -> 12288, down 12288 -> 3072 (Q6_K on the image stream, Q4_K on the text stream).
CONFIG3 = [("qk", Q4K, 6144, 3072), ("v", Q6K, 3072, 3072), ("out", Q4K, 3072, 3072), ("up", Q4K, 12288, 3072)]


@pytest.mark.parametrize("m,stream", [(1024, "image"), (4096, "image"), (256, "text")])
def test_config3_stream_linears(mods, m, stream):
    rows = sample_rows(m, 400 + m)
    down_type = Q6K if stream == "image" else Q4K
    for i, (name, typ, n, k) in enumerate(CONFIG3 + [("down", down_type, 3072, 12288)]):
        run_projection(mods, f"config3 {stream} {name}", typ, n, k, m, 310 + 10 * i, rows)


def test_config3_adaln_modulation_m1(mods):
    """adaLN modulation 3072 -> 18432 (6 x hidden) at M = 1, with a bias: every output."""
    run_projection(mods, "config3 adaLN", Q4K, 18432, 3072, 1, 390)


# ---- config 4: LTX video DiT, hidden 4096, MLP 16384, 4132 tokens ----------------------------
CONFIG4 = [("qkv", Q4K, 12288, 4096), ("out", Q6K, 4096, 4096), ("ff_up", Q4K, 16384, 4096),
           ("ff_down", Q6K, 4096, 16384)]


def test_config4_video_linears(mods):
    """4132 tokens = 16 full 256-row tiles + 36 rows on the skinny kernel: sampled rows
    include every tail row's neighbourhood."""
    m = 4132
    rows = sample_rows(m, 500, extra=range(4096, 4132))
    for i, (name, typ, n, k) in enumerate(CONFIG4):
        run_projection(mods, f"config4 {name}", typ, n, k, m, 510 + 10 * i, rows)


def test_config4_cross_attention_kv_m128(mods):
    run_projection(mods, "config4 cross-attn kv", Q4K, 8192, 4096, 128, 560)


@pytest.mark.parametrize("typ,n,k,seed", [(Q6K, 4096, 16384, 570),   # config 4 ff_down
                                           (Q6K, 3072, 12288, 580)])  # config 3 image-stream down
def test_long_k_q6k_one_hot_exact(mods, typ, n, k, seed):
    """One-hot activation rows e_r (r < k) at the full long-K Q6_K shapes: y[r] is column r of
    the weight, i.e. y^T equals the bf16-decoded weight matrix bit for bit (the device decode,
    itself bit-exact to the oracle, test_gpu_decode.py); the full matrix is also checked on
    the CPU for a band of rows."""
    gguf, ql = mods
    blocks, raw = dev_weight(gguf, typ, n, k, seed)
    lin = ql.QuantizedLinear(blocks, typ, n, k)
    x = torch.zeros((k, k), dtype=torch.bfloat16, device="cuda")
    x[torch.arange(k), torch.arange(k)] = 1.0
    print(f"[one-hot long K] type={typ} n={n} k={k}", flush=True)
    y = lin(x)
    wb = gguf.dequantize(blocks, typ, n, k, gguf.DecodeDType.bf16)
    got = y.t().contiguous().view(torch.int16)
    want = wb.view(torch.int16)
    zg, zw = (got & 0x7FFF) == 0, (want & 0x7FFF) == 0
    assert torch.equal(zg, zw) and torch.equal(got[~zg], want[~zw])
    band = slice(n // 2, n // 2 + 64)
    assert np.array_equal(host_bf16(wb[band]), oracle.decode_matrix(raw, typ, n, k, dtype=oracle.DTYPE_BF16)[band])


# ---- config 5: runtime LoRA per image at config-3 shapes ------------------------------------
@pytest.mark.parametrize("n,ranks", [(3072, (16, 64, 16, 64)), (12288, (64, 16, 64, 16))])
def test_config5_per_image_lora(mods, n, ranks):
    """4 images x 1280 tokens (M = 5120), K = 3072; image i carries adapter i: A [r, 3072] bf16
    N(0, 1/r), B [n, r] bf16 N(0, 0.01), strength U[0.5, 1.5], no alpha (scale = strength);
    bias last. Sampled rows of every image against the reference's runtime-LoRA sequence
    (mlx.cpp:692-722) per image."""
    gguf, ql = mods
    per, k = 1280, 3072
    m = 4 * per
    blocks, raw = dev_weight(gguf, Q4K, n, k, 600 + n)
    bias = dev_bias(n, 601)
    lin = ql.QuantizedLinear(blocks, Q4K, n, k, bias)
    x = dev_x(m, k, 602)
    rng = np.random.default_rng(700)
    adapters, host_ads = [], []
    for i, r in enumerate(ranks):
        a = oracle.bf16_bits((rng.standard_normal((r, k)) / r).astype(np.float32))
        b = oracle.bf16_bits((rng.standard_normal((n, r)) * 0.01).astype(np.float32))
        s = ql.lora_scale(float(rng.uniform(0.5, 1.5)), r)
        ta = torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
        tb = torch.from_numpy(b.view(np.int16)).cuda().view(torch.bfloat16)
        adapters.append(ql.LoRAAdapter(ta, tb, s, i * per, per))
        host_ads.append((a, b, s))
    print(f"[config5] n={n} ranks={ranks}", flush=True)
    y = lin(x, adapters)
    base = ql.QuantizedLinear(blocks, Q4K, n, k)(x)   # the same base launch, no bias, no adapters
    torch.cuda.synchronize()
    rows = sample_rows(m, 703, extra=[i * per + j for i in range(4) for j in (0, 1, per - 1)])
    sel = torch.from_numpy(rows).cuda()
    xh, yh, bh = host_bf16(x[sel]), host_bf16(y[sel]), host_bf16(base[sel])
    sampled_ads = []
    for i, (a, b, s) in enumerate(host_ads):
        own = np.flatnonzero((rows >= i * per) & (rows < (i + 1) * per))
        sampled_ads.append(dict(a=a, b=b, scale=s, row_begin=int(own[0]), row_count=int(own.size)))
    wb = oracle_weights(raw, Q4K, n, k, m)
    check_lora(f"config5 n={n}", yh, bh, xh, wb, bias.cpu().numpy(), sampled_ads)
    # The adapters matter: the base projection alone is far from the result.
    plain = oracle.add_bias(oracle.linear_reference(xh, wb), oracle.bias_to_bf16(bias.cpu().numpy()))
    assert oracle.compare_bf16(yh, plain)["max_abs"] > 1e-2


@pytest.mark.parametrize("typ", [Q4K, 13, Q6K])
@pytest.mark.parametrize("m,n", [(1024, 6144), (2048, 5120)])
def test_runtime_lora_on_unsplit_gemm(mods, typ, m, n):
    """With adapters bound, an unsplit GEMM writes y with cached stores (the LoRA pass reads it
    back at once), without adapters with non-temporal ones: 128-row tiles at 1024 x 6144,
    256-row tiles at 2048 x 5120 (K = 3072, both unsplit). An adapter whose B is zero must
    leave the adapter-free output unchanged; two real adapters on the two halves of the rows
    match the oracle on sampled rows."""
    gguf, ql = mods
    k = 3072
    if typ == 13:  # no device quantizer for Q5_K: random codes under small scales, uploaded
        from test_gpu_qlinear import dense_type_payload
        raw = dense_type_payload(13, n, k, np.random.default_rng(800))
        blocks = torch.from_numpy(raw).cuda()
    else:
        blocks, raw = dev_weight(gguf, typ, n, k, 800 + typ)
    lin = ql.QuantizedLinear(blocks, typ, n, k)
    x = dev_x(m, k, 801)
    print(f"[lora unsplit gemm] type={typ} m={m} n={n}", flush=True)
    base = lin(x)
    a0 = torch.full((16, k), 0.01, device="cuda").to(torch.bfloat16)
    b0 = torch.zeros((n, 16), device="cuda").to(torch.bfloat16)
    y0 = lin(x, [ql.LoRAAdapter(a0, b0, 1.0, 0, m)])
    torch.cuda.synchronize()
    assert torch.equal(y0, base)
    rng = np.random.default_rng(802)
    half = m // 2
    adapters, host_ads = [], []
    for i, r in enumerate((16, 64)):
        a = oracle.bf16_bits((rng.standard_normal((r, k)) / r).astype(np.float32))
        b = oracle.bf16_bits((rng.standard_normal((n, r)) * 0.01).astype(np.float32))
        s = ql.lora_scale(float(rng.uniform(0.5, 1.5)), r)
        ta = torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
        tb = torch.from_numpy(b.view(np.int16)).cuda().view(torch.bfloat16)
        adapters.append(ql.LoRAAdapter(ta, tb, s, i * half, half))
        host_ads.append((a, b, s))
    y = lin(x, adapters)
    torch.cuda.synchronize()
    rows = sample_rows(m, 803, extra=[half - 1, half])
    sel = torch.from_numpy(rows).cuda()
    xh, yh, bh = host_bf16(x[sel]), host_bf16(y[sel]), host_bf16(base[sel])
    sampled_ads = []
    for i, (a, b, s) in enumerate(host_ads):
        own = np.flatnonzero((rows >= i * half) & (rows < (i + 1) * half))
        sampled_ads.append(dict(a=a, b=b, scale=s, row_begin=int(own[0]), row_count=int(own.size)))
    check_lora(f"lora unsplit gemm t{typ} {m}x{n}", yh, bh, xh, oracle_weights(raw, typ, n, k, m), None, sampled_ads)


def test_bind_runtime_lora_with_alpha_scale(mods):
    """Weights.bind_runtime_lora with alpha 3, rank 20, strength 0.3: the effective scale is the
    reference's two fp32 roundings (mlx.cpp:1442-1452), which the device applies."""
    gguf, ql = mods
    n, k, m, r = 3072, 3072, 64, 20
    blocks, raw = dev_weight(gguf, Q4K, n, k, 800)
    bias = dev_bias(n, 801)
    w = ql.Weights()
    w.bind("blk.attn_out", blocks, Q4K, n, k, bias)
    rng = np.random.default_rng(802)
    a = oracle.bf16_bits((rng.standard_normal((r, k)) / r).astype(np.float32))
    b = oracle.bf16_bits((rng.standard_normal((n, r)) * 0.05).astype(np.float32))
    w.bind_runtime_lora("blk.attn_out", torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16),
                        torch.from_numpy(b.view(np.int16)).cuda().view(torch.bfloat16), 0.3, alpha=3.0)
    scale = np.float32(np.float32(0.3) * np.float32(np.float32(3.0) / np.float32(r)))
    assert w._runtime["blk.attn_out"][0].scale == float(scale)
    x = dev_x(m, k, 803)
    y = w.project(x, "blk.attn_out")
    base = ql.QuantizedLinear(blocks, Q4K, n, k)(x)
    torch.cuda.synchronize()
    check_lora("bind alpha", host_bf16(y), host_bf16(base), host_bf16(x), oracle_weights(raw, Q4K, n, k, m),
               bias.cpu().numpy(), [dict(a=a, b=b, scale=float(scale))])
