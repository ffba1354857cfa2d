"""GPU: stacked projections (Weights.bind_stacked / project_stacked), the batched adaLN
modulation of a DiT: every block's modulation projection reads the same timestep embedding,
so their rows run as one launch (native/models/qwen21/transformer.cpp:617).

Each member's columns of the stacked output must match the oracle for that member alone (the
one-row GEMV's exact-weight route at 1-2 rows, the bf16-decode route above), members keep
projecting on their own from views of the stacked rows, and runtime adapters bound to a
member apply to its columns only.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from parity import check, check_lora, expect
from test_gpu_qlinear import activations, from_dev_bf16, to_dev_bf16, weights

pytestmark = pytest.mark.gpu

Q4K, Q6K = 12, 14
SIZES = [3072, 2048, 512, 1024, 768]


def _bind(ql, typ, k, seed, bias=True):
    rng = np.random.default_rng(seed)
    W = ql.Weights()
    members = {}
    for i, n in enumerate(SIZES):
        blocks = weights(typ, n, k, seed + i)
        b = (rng.standard_normal(n) * 0.1).astype(np.float32) if bias else None
        W.bind(f"blocks.{i}.mod", torch.from_numpy(blocks).cuda(), typ, n, k,
               torch.from_numpy(b).cuda() if b is not None else None)
        members[f"blocks.{i}.mod"] = (blocks, b, n)
    return W, members


def _want(x, blocks, typ, n, k, b, m):
    route = "exact" if m <= 8 else "bf16"
    w = (oracle.decode_matrix(blocks, typ, n, k) if route == "exact"
         else oracle.bf16_to_f32(oracle.decode_matrix(blocks, typ, n, k, dtype=oracle.DTYPE_BF16)))
    return w, route


@pytest.mark.parametrize("typ,m", [(Q4K, 1), (Q6K, 1), (Q4K, 2), (Q4K, 40)])
def test_stacked_members_match_oracle(ql, typ, m):
    k = 1024
    W, members = _bind(ql, typ, k, 300 + m)
    W.bind_stacked("mod.all", list(members))
    x = activations(m, k, 301, scale=1.0)
    xd = to_dev_bf16(x)
    print(f"[stacked] type={typ} m={m} rows={sum(SIZES)}", flush=True)
    outs = W.project_stacked(xd, "mod.all")
    torch.cuda.synchronize()
    assert list(outs) == list(members)
    for p, (blocks, b, n) in members.items():
        got = from_dev_bf16(outs[p].contiguous())
        w, route = _want(x, blocks, typ, n, k, b, m)
        check(f"stacked {p}", got, *expect(x, w, b), route=route)
        # The member alone, from its view of the stacked rows.
        alone = from_dev_bf16(W.project(xd, p))
        check(f"member {p}", alone, *expect(x, w, b), route=route)


@pytest.fixture(scope="module")
def ql():
    from turbocider_amd import qlinear
    return qlinear


def test_stacked_with_member_lora(ql):
    k, m, r = 1024, 2, 8
    W, members = _bind(ql, Q4K, k, 320)
    rng = np.random.default_rng(321)
    target = "blocks.2.mod"
    n = members[target][2]
    a = oracle.bf16_bits((rng.standard_normal((r, k)) * 0.05).astype(np.float32))
    bb = oracle.bf16_bits((rng.standard_normal((n - 100, r)) * 0.05).astype(np.float32))
    W.bind_stacked("mod.all", list(members))
    W.bind_runtime_lora(target, to_dev_bf16(a), to_dev_bf16(bb), 0.8, alpha=16.0, output_start=50,
                        output_end=n - 50)
    with pytest.raises(ql.QLinearError, match="members"):
        W.bind_runtime_lora("mod.all", to_dev_bf16(a), to_dev_bf16(bb), 1.0)
    x = activations(m, k, 322)
    xd = to_dev_bf16(x)
    print("[stacked] member lora", flush=True)
    outs = W.project_stacked(xd, "mod.all")
    torch.cuda.synchronize()
    scale = ql.lora_scale(0.8, r, 16.0)
    for p, (blocks, b, nn) in members.items():
        got = from_dev_bf16(outs[p].contiguous())
        w, route = _want(x, blocks, Q4K, nn, k, b, m)
        if p == target:
            ads = [dict(a=a, b=bb, scale=scale, out_begin=50, out_end=nn - 50)]
            want, chain = oracle.linear_reference_chain(x, w, oracle.bias_to_bf16(b), ads)
            check(f"stacked lora {p}", got, want, chain, tight=False)
        else:
            check(f"stacked {p}", got, *expect(x, w, b), route=route)


def test_stack_errors(ql):
    k = 512
    W = ql.Weights()
    W.bind("a", torch.from_numpy(weights(Q4K, 256, k, 1)).cuda(), Q4K, 256, k)
    W.bind("b", torch.from_numpy(weights(Q6K, 256, k, 2)).cuda(), Q6K, 256, k)
    W.bind("c", torch.from_numpy(weights(Q4K, 256, k, 3)).cuda(), Q4K, 256, k,
           torch.zeros(256, device="cuda"))
    with pytest.raises(ql.QLinearError, match="share the weight type"):
        W.bind_stacked("s", ["a", "b"])
    with pytest.raises(ql.QLinearError, match="all have a bias or none"):
        W.bind_stacked("s", ["a", "c"])
    with pytest.raises(ql.QLinearError, match="distinct"):
        W.bind_stacked("s", ["a", "a"])
    with pytest.raises(ql.QLinearError, match="missing weight"):
        W.bind_stacked("s", ["a", "zz"])
