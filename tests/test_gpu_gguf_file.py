"""GPU: GGUF file -> raw blocks in HBM -> projection, against the oracle.

A file written with Q4_K and Q6_K weights (``blk.N.*`` and ``model.diffusion_model.*``
names, an F32 bias, alignment 64) is opened with the container reader; every payload that
lands in device memory must equal the file bytes, and the bound projections must match the
oracle's bf16-decode route (tolerance as the other GEMM tests).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from test_gguf_file import STRING, U32, image, kv

pytestmark = pytest.mark.gpu

Q4K, Q6K = 12, 14


def test_gguf_file_upload_and_projection(tmp_path):
    from turbocider_amd import gguf_file, qlinear
    rng = np.random.default_rng(90)
    wq = oracle.quantize(Q4K, (rng.standard_normal((300, 512)) * 0.02).astype(np.float32))
    wd = oracle.quantize(Q6K, (rng.standard_normal((256, 768)) * 0.02).astype(np.float32))
    bias = (rng.standard_normal(300) * 0.01).astype(np.float32)
    raw = image(("model.diffusion_model.blocks.0.attn.to_q.weight", Q4K, [512, 300], None, wq.tobytes()),
                ("model.diffusion_model.blocks.0.attn.to_q.bias", 0, [300], None, bias.tobytes()),
                ("blocks.0.ff.down.weight", Q6K, [768, 256], None, wd.tobytes()),
                pairs=[kv("general.alignment", U32, 64), kv("general.architecture", STRING, "qwen_image")],
                alignment=64).build()
    path = tmp_path / "tiny.gguf"
    path.write_bytes(raw)
    print("[gguf] upload", flush=True)
    with gguf_file.GGUFFile(path) as f:
        assert f.projection_prefixes() == ["blocks.0.attn.to_q", "blocks.0.ff.down"]
        got = f.read_tensor("blocks.0.ff.down.weight").cpu().numpy()
        assert np.array_equal(got, wd.reshape(-1))
        W = qlinear.Weights()
        for p in f.projection_prefixes():
            f.bind_projection(W, p)
    for prefix, blocks, typ, n, k, b in (("blocks.0.attn.to_q", wq, Q4K, 300, 512, bias),
                                         ("blocks.0.ff.down", wd, Q6K, 256, 768, None)):
        for m in (1, 40, 300):
            print(f"[gguf] project {prefix} m={m}", flush=True)
            x = oracle.bf16_bits((rng.standard_normal((m, k))).astype(np.float32))
            y = W.project(torch.from_numpy(x.view(np.int16)).cuda().view(torch.bfloat16), prefix)
            torch.cuda.synchronize()
            y = y.cpu().view(torch.int16).numpy().view(np.uint16)
            wb = oracle.bf16_to_f32(oracle.decode_matrix(blocks, typ, n, k, dtype=oracle.DTYPE_BF16))
            wf = oracle.decode_matrix(blocks, typ, n, k)
            bb = oracle.bias_to_bf16(b) if b is not None else None
            want = oracle.linear_reference(x, wf if m == 1 else wb, bb)
            stats = oracle.compare_bf16(y, want)
            assert oracle.within_tolerance(stats, y, want), (prefix, m, stats)


def test_gguf_embedding_row_gather(tmp_path):
    """A prompt's token rows of an embedding table (Q8_0 / BF16 / Q4_K / Q6_K) gathered and
    decoded on the device equal the reference decoder's gather (the oracle, pinned to it)."""
    from turbocider_amd import gguf_file
    rng = np.random.default_rng(91)
    vocab, hidden = 1000, 512
    tables = {}
    q8 = rng.integers(0, 256, size=vocab * hidden // 32 * 34, dtype=np.uint8).reshape(-1, 34)
    q8[:, 0:2] = np.frombuffer(np.float16(0.001).tobytes() * len(q8), dtype=np.uint8).reshape(-1, 2)
    tables[8] = q8.reshape(-1)
    tables[30] = oracle.bf16_bits((rng.standard_normal(vocab * hidden) * 0.02).astype(np.float32)).view(np.uint8)
    tables[12] = oracle.quantize(12, (rng.standard_normal((vocab, hidden)) * 0.02).astype(np.float32))
    tables[14] = oracle.quantize(14, (rng.standard_normal((vocab, hidden)) * 0.02).astype(np.float32))
    names = {t: f"token_embd_{t}.weight" for t in tables}
    raw = image(*[(names[t], t, [hidden, vocab], None, tables[t].tobytes()) for t in tables],
                pairs=[kv("general.alignment", U32, 32)]).build()
    path = tmp_path / "embd.gguf"
    path.write_bytes(raw)
    ids = [5, 999, 0, 5, 417]
    with gguf_file.GGUFFile(path) as f:
        for t in tables:
            print(f"[gguf] gather type={t}", flush=True)
            got = f.gather_rows(names[t], ids).cpu().view(torch.int16).numpy().view(np.uint16)
            st, want, _, err = oracle.decode_raw(tables[t].tobytes(), t, vocab, hidden, gather=ids, dtype=2)
            assert st == 0, err
            assert np.array_equal(got, np.frombuffer(want, dtype=np.uint16).reshape(len(ids), hidden)), t


def test_gguf_load_projections_all_or_nothing(tmp_path):
    """load_projections on the device: a bad third projection (bias of the wrong length) binds
    nothing; the good file binds every projection, and each matches bind_projection's."""
    from turbocider_amd import _lib, gguf_file, qlinear
    rng = np.random.default_rng(92)
    w = [oracle.quantize(Q4K, (rng.standard_normal((256, 512)) * 0.02).astype(np.float32)) for _ in range(3)]
    good_bias = (rng.standard_normal(256) * 0.01).astype(np.float32)
    tensors = [(f"p{i}.weight", Q4K, [512, 256], None, w[i].tobytes()) for i in range(3)]
    bad = image(*tensors, ("p2.bias", 0, [255], None, good_bias[:255].tobytes())).build()
    good = image(*tensors, ("p2.bias", 0, [256], None, good_bias.tobytes())).build()
    (tmp_path / "bad.gguf").write_bytes(bad)
    (tmp_path / "good.gguf").write_bytes(good)
    print("[gguf] load_projections bad", flush=True)
    with gguf_file.GGUFFile(tmp_path / "bad.gguf") as f:
        W = qlinear.Weights()
        with pytest.raises(_lib.NativeError, match="255 values for 256 outputs"):
            f.load_projections(W)
        assert W.bound_prefixes() == []
    print("[gguf] load_projections good", flush=True)
    with gguf_file.GGUFFile(tmp_path / "good.gguf") as f:
        W = qlinear.Weights()
        assert f.load_projections(W) == ["p0", "p1", "p2"]
        W1 = qlinear.Weights()
        for p in ("p0", "p1", "p2"):
            f.bind_projection(W1, p)
    x = torch.from_numpy(oracle.bf16_bits(rng.standard_normal((40, 512)).astype(np.float32)).view(np.int16))
    x = x.cuda().view(torch.bfloat16)
    for p in ("p0", "p1", "p2"):
        a, b = W.project(x, p), W1.project(x, p)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), p
