"""GPU: projections with an output activation (tc_qlinear_forward_act), fused MLPs and gate_up
bindings, against the oracle.

The activation is a function of the projection's finished bf16 outputs, so each route is
checked in two parts:
* the same projection without the activation (same handle, same route, same summation order)
  gives `pre`, which the other tests check against the oracle GEMM;
* the activated output must equal oracle.act_reference(pre) (float64, one rounding), except
  that an output may differ by one bf16 ulp where the fp32 evaluation and the float64 value
  fall on the two sides of a rounding boundary: at most 0.1 % of outputs.
Every kernel route is covered: the GEMM unsplit (activation in its epilogue), split K (in the
slice reduction), with skinny tail rows, the skinny kernel unsplit and split, the one-row and
2..8-row GEMVs, and the routes that apply it as a second pass (forced per-row GEMV, runtime
LoRA, the library GEMM of other types).
"""
from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

from oracle import oracle
from parity import check, expect
from test_gpu_qlinear import activations, dense_type_payload, from_dev_bf16, to_dev_bf16, weights
from test_plan import DENSE, GEMM, GEMV, GEMV1, GEMV8, SKINNY, plan

pytestmark = pytest.mark.gpu

Q4K, Q6K = 12, 14
GELU, GLU = "gelu_tanh", "silu_glu"
ACT_CODE = {GELU: oracle.ACT_GELU_TANH, GLU: oracle.ACT_SILU_GLU}


def check_act(name, got, pre, act, max_fraction=1e-3):
    want = oracle.act_reference(pre, ACT_CODE[act])
    assert got.shape == want.shape, (name, got.shape, want.shape)
    g = oracle.bf16_to_f32(got).astype(np.float64)
    w = oracle.bf16_to_f32(want).astype(np.float64)
    differ = got != want
    # Both +0 and -0 are zeros of the activation; any other difference is at most one ulp.
    differ &= ~((g == 0) & (w == 0))
    # One bf16 ulp at the larger magnitude (subnormals: the fixed spacing 2^-133).
    ulp = np.maximum(np.ldexp(1.0, np.frexp(np.maximum(np.abs(g), np.abs(w)))[1] - 8), 2.0 ** -133)
    within = np.abs(g - w) <= ulp
    n_diff = int(differ.sum())
    print(f"[{name}] {act}: {n_diff} of {got.size} outputs differ by one ulp", flush=True)
    for i in np.flatnonzero((differ & ~within).reshape(-1))[:8]:
        src = pre.reshape(-1)[i] if act == GELU else pre.reshape(pre.shape[0], -1, 2).reshape(-1, 2)[i]
        print(f"[{name}] beyond one ulp at {i}: pre {src} got {g.reshape(-1)[i]!r} want {w.reshape(-1)[i]!r}",
              flush=True)
    assert np.all(within | ~differ), (name, act, "more than one ulp")
    assert n_diff <= oracle.allowed_differing(got.size, max_fraction), (name, act, n_diff)


def run(lin, x, act=None, adapters=()):
    y = lin(to_dev_bf16(x), adapters, act=act)
    torch.cuda.synchronize()
    return from_dev_bf16(y)


def linear(ql, blocks, typ, n, k, bias=None, path=0):
    lin = ql.QuantizedLinear(torch.from_numpy(blocks).cuda(), typ, n, k,
                             torch.from_numpy(bias).cuda() if bias is not None else None)
    lin.set_path(path)
    return lin


@pytest.fixture(scope="module")
def ql():
    from turbocider_amd import qlinear
    return qlinear


# (name, type, m, n, k, path, expected kernel, split K expected)
ROUTES = [
    ("gemm unsplit", Q4K, 1024, 6144, 512, 0, GEMM, False),
    ("gemm split", Q4K, 256, 512, 4096, 0, GEMM, True),
    ("gemm + skinny tail", Q6K, 2600, 6400, 512, 0, GEMM, None),
    ("skinny unsplit", Q4K, 40, 10240, 512, 0, SKINNY, False),
    ("skinny split", Q6K, 40, 512, 4096, 0, SKINNY, True),
    ("gemv1", Q4K, 1, 4096, 1024, 0, GEMV1, None),
    ("gemv1 q6k", Q6K, 1, 2048, 1024, 0, GEMV1, None),
    ("gemv8", Q6K, 5, 2048, 1024, 0, GEMV8, None),
    ("forced per-row gemv (second pass)", Q4K, 3, 512, 512, 2, GEMV, None),
]


@pytest.mark.parametrize("name,typ,m,n,k,path,kernel,split", ROUTES, ids=[r[0] for r in ROUTES])
@pytest.mark.parametrize("act", [GELU, GLU])
def test_activation_routes(ql, name, typ, m, n, k, path, kernel, split, act):
    st, info, text = plan(typ, n, k, m, path=path)
    assert st == 0 and info.kernel == kernel, (name, info.kernel, text)
    if split is not None:
        assert (info.workspace_bytes > 0) == split, (name, info.workspace_bytes)
    if name == "gemm + skinny tail":
        assert info.tail_rows > 0
    rng = np.random.default_rng(zlib.crc32(f"{name}/{act}".encode()))
    blocks = weights(typ, n, k, 10 + m)
    bias = (rng.standard_normal(n) * 0.5).astype(np.float32)
    x = activations(m, k, 20 + m, scale=2.0)
    lin = linear(ql, blocks, typ, n, k, bias, path)
    print(f"[act] {name} {act} m={m} n={n} k={k}", flush=True)
    pre = run(lin, x)
    h = run(lin, x, act)
    check_act(name, h, pre, act)
    # A second call reuses the handle's workspaces and gives the same bits.
    assert np.array_equal(run(lin, x, act), h)


@pytest.mark.parametrize("act", [GELU, GLU])
def test_activation_with_runtime_lora(ql, act):
    """Adapters (and the bias after them) finish the outputs first; the activation follows as a
    second pass on the same bits."""
    m, n, k, r = 48, 768, 512, 16
    rng = np.random.default_rng(31)
    blocks = weights(Q4K, n, k, 32)
    bias = (rng.standard_normal(n) * 0.5).astype(np.float32)
    x = activations(m, k, 33)
    lin = linear(ql, blocks, Q4K, n, k, bias)
    a = to_dev_bf16(oracle.bf16_bits((rng.standard_normal((r, k)) * 0.05).astype(np.float32)))
    b = to_dev_bf16(oracle.bf16_bits((rng.standard_normal((n - 64, r)) * 0.05).astype(np.float32)))
    ads = [ql.LoRAAdapter(a, b, 0.75, 0, None, 32, n - 32)]
    print(f"[act] lora {act}", flush=True)
    pre = run(lin, x, adapters=ads)
    h = run(lin, x, act, adapters=ads)
    check_act("lora", h, pre, act)


@pytest.mark.parametrize("act", [GELU, GLU])
def test_activation_on_library_gemm_route(ql, act):
    m, n, k = 24, 512, 512
    rng = np.random.default_rng(41)
    raw = dense_type_payload(8, n, k, rng)
    st, info, _ = plan(8, n, k, m)
    assert st == 0 and info.kernel == DENSE
    lin = linear(ql, raw, 8, n, k)
    x = activations(m, k, 42)
    print(f"[act] dense Q8_0 {act}", flush=True)
    pre = run(lin, x)
    h = run(lin, x, act)
    check_act("dense", h, pre, act)


def test_activation_argument_errors(ql):
    blocks = weights(Q4K, 258, 512, 5)
    odd = linear(ql, weights(Q4K, 257, 512, 6), Q4K, 257, 512)
    x = to_dev_bf16(activations(4, 512, 7))
    with pytest.raises(ql.QLinearError, match="even number of outputs"):
        odd(x, act=GLU)
    with pytest.raises(ql.QLinearError, match="unknown output activation"):
        odd(x, act="relu")
    lin = linear(ql, blocks, Q4K, 258, 512)
    with pytest.raises(ql.QLinearError, match=r"\[m, 129\]"):
        lin(x, out=torch.empty((4, 258), dtype=torch.bfloat16, device="cuda"), act=GLU)
    with pytest.raises(ql.QLinearError, match="allocation-free"):
        lin(x, act=GELU, allocation_free=True)


def _gate_up(ql, typ, n, k, seed, bias=True):
    """A gate_up weight in the reference's [gate; up] row order, bound with bind_gate_up."""
    rng = np.random.default_rng(seed)
    blocks = weights(typ, 2 * n, k, seed)
    b = (rng.standard_normal(2 * n) * 0.5).astype(np.float32) if bias else None
    W = ql.Weights()
    W.bind_gate_up("mlp.gate_up", torch.from_numpy(blocks).cuda(), typ, 2 * n, k,
                   torch.from_numpy(b).cuda() if b is not None else None)
    return W, blocks, b


@pytest.mark.parametrize("typ,m", [(Q4K, 1), (Q4K, 6), (Q6K, 40), (Q4K, 300)])
def test_gate_up_binding_projects_in_reference_order(ql, typ, m):
    """project() of a gate_up binding returns [gate; up] columns matching the oracle, and
    project_act(..., "silu_glu") equals silu(gate) * up of those same bits."""
    n, k = 1024, 512
    W, blocks, b = _gate_up(ql, typ, n, k, 50 + m)
    x = activations(m, k, 51 + m, scale=2.0)
    xd = to_dev_bf16(x)
    print(f"[gate_up] type={typ} m={m}", flush=True)
    y = W.project(xd, "mlp.gate_up")
    h = W.project_act(xd, "mlp.gate_up", GLU)
    torch.cuda.synchronize()
    y, h = from_dev_bf16(y), from_dev_bf16(h)
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, typ, 2 * n, k, dtype=oracle.DTYPE_BF16))
    wf = oracle.decode_matrix(blocks, typ, 2 * n, k)
    route = "exact" if m <= 8 else "bf16"
    check(f"gate_up m={m}", y, *expect(x, wf if route == "exact" else wb, b), route=route)
    inter = np.empty_like(y)
    inter[:, 0::2], inter[:, 1::2] = y[:, :n], y[:, n:]
    check_act(f"gate_up m={m}", h, inter, GLU)


def test_gate_up_runtime_lora_in_reference_order(ql):
    """An adapter bound in the reference's column order (a range across the gate/up boundary)
    lands on the right interleaved rows."""
    n, k, m, r = 512, 512, 24, 8
    W, blocks, b = _gate_up(ql, Q4K, n, k, 60)
    rng = np.random.default_rng(61)
    ob, oe = 300, 800  # gate columns 300..511 and up columns 0..287
    a = oracle.bf16_bits((rng.standard_normal((r, k)) * 0.05).astype(np.float32))
    bb = oracle.bf16_bits((rng.standard_normal((oe - ob, r)) * 0.05).astype(np.float32))
    W.bind_runtime_lora("mlp.gate_up", to_dev_bf16(a), to_dev_bf16(bb), 1.25, alpha=4.0, output_start=ob,
                        output_end=oe)
    x = activations(m, k, 62)
    print("[gate_up] lora", flush=True)
    y = W.project(to_dev_bf16(x), "mlp.gate_up")
    torch.cuda.synchronize()
    y = from_dev_bf16(y)
    wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, Q4K, 2 * n, k, dtype=oracle.DTYPE_BF16))
    scale = ql.lora_scale(1.25, r, 4.0)
    ads = [dict(a=a, b=bb, scale=scale, out_begin=ob, out_end=oe)]
    want, chain = oracle.linear_reference_chain(x, wb, oracle.bias_to_bf16(b), ads)
    check("gate_up lora end to end", y, want, chain, tight=False)


@pytest.mark.parametrize("m", [1, 40, 512])
def test_mlp_silu_glu_then_down(ql, m):
    """project_mlp on a gate_up binding: h = silu(gate) * up from the epilogue, then the down
    projection of h, each against the oracle (down on the kernel's own h)."""
    n, k = 1536, 512
    W, blocks, b = _gate_up(ql, Q4K, n, k, 70 + m)
    dblocks = weights(Q6K, k, n, 71 + m)
    W.bind("mlp.down", torch.from_numpy(dblocks).cuda(), Q6K, k, n)
    x = activations(m, k, 72 + m)
    xd = to_dev_bf16(x)
    print(f"[mlp] silu_glu m={m}", flush=True)
    out = W.project_mlp(xd, "mlp.gate_up", "mlp.down")
    y = W.project(xd, "mlp.gate_up")
    h = W.project_act(xd, "mlp.gate_up", GLU)
    torch.cuda.synchronize()
    out, y, h = from_dev_bf16(out), from_dev_bf16(y), from_dev_bf16(h)
    inter = np.empty_like(y)
    inter[:, 0::2], inter[:, 1::2] = y[:, :n], y[:, n:]
    check_act(f"mlp h m={m}", h, inter, GLU)
    route = "exact" if m <= 8 else "bf16"
    dw = (oracle.decode_matrix(dblocks, Q6K, k, n) if route == "exact"
          else oracle.bf16_to_f32(oracle.decode_matrix(dblocks, Q6K, k, n, dtype=oracle.DTYPE_BF16)))
    check(f"mlp down m={m}", out, *expect(h, dw), route=route)


@pytest.mark.parametrize("m", [1, 300])
def test_mlp_gelu_then_down(ql, m):
    """The MMDiT MLP: up (Q4_K, bias) -> GELU in the epilogue -> down (Q6_K)."""
    n, k = 2048, 512
    rng = np.random.default_rng(80 + m)
    ub = weights(Q4K, n, k, 81 + m)
    bias = (rng.standard_normal(n) * 0.5).astype(np.float32)
    dblocks = weights(Q6K, k, n, 82 + m)
    W = ql.Weights()
    W.bind("ff.up", torch.from_numpy(ub).cuda(), Q4K, n, k, torch.from_numpy(bias).cuda())
    W.bind("ff.down", torch.from_numpy(dblocks).cuda(), Q6K, k, n)
    x = activations(m, k, 83 + m, scale=2.0)
    xd = to_dev_bf16(x)
    print(f"[mlp] gelu m={m}", flush=True)
    out = W.project_mlp(xd, "ff.up", "ff.down")
    pre = W.project(xd, "ff.up")
    torch.cuda.synchronize()
    out, pre = from_dev_bf16(out), from_dev_bf16(pre)
    h = oracle.act_reference(pre, oracle.ACT_GELU_TANH)
    route = "exact" if m <= 8 else "bf16"
    dw = (oracle.decode_matrix(dblocks, Q6K, k, n) if route == "exact"
          else oracle.bf16_to_f32(oracle.decode_matrix(dblocks, Q6K, k, n, dtype=oracle.DTYPE_BF16)))
    # The down projection of the oracle's h: the kernel's h may differ from it by rare 1-ulp
    # activation roundings, which the north-star bound absorbs.
    check(f"mlp gelu m={m}", out, *expect(h, dw), route=route, tight=False)
