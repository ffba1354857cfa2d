"""GPU: the weight pager (tc_pager_*, gguf_file.GGUFPager) streams groups of projections from a
GGUF file through a bounded set of device slots.

The reference pages blocks of a model that does not fit in memory through a slot pool
(native/runtime/streaming/gguf_weight_pager.hpp:27-53, slot_pool.hpp:11-45). Here: a file of
six blocks (a Q4_K projection with an F32 bias and a Q6_K projection each) goes through two
and three slots; every block's outputs must equal those of the same projections bound
resident (bind_projection: identical bytes, identical kernels, so identical bits), and the
resident outputs are checked against the oracle. Also: the slot protocol's errors (fill into a
slot in use, stale tickets, release before bind), cancellation, and a file that changes
under the pager.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import oracle
from parity import check, expect
from test_gguf_file import U32, image, kv
from test_gpu_qlinear import activations, from_dev_bf16, to_dev_bf16

pytestmark = pytest.mark.gpu

Q4K, Q6K = 12, 14
BLOCKS, K, N_Q, N_D = 6, 512, 768, 512


def _model(tmp_path, seed=5):
    rng = np.random.default_rng(seed)
    tensors, want = [], {}
    for b in range(BLOCKS):
        wq = oracle.quantize(Q4K, (rng.standard_normal((N_Q, K)) * 0.02).astype(np.float32))
        bq = (rng.standard_normal(N_Q) * 0.05).astype(np.float32)
        wd = oracle.quantize(Q6K, (rng.standard_normal((N_D, N_Q)) * 0.02).astype(np.float32))
        tensors += [(f"blk.{b}.attn_q.weight", Q4K, [K, N_Q], None, wq.tobytes()),
                    (f"blk.{b}.attn_q.bias", 0, [N_Q], None, bq.tobytes()),
                    (f"blk.{b}.ffn_down.weight", Q6K, [N_Q, N_D], None, wd.tobytes())]
        want[b] = (wq, bq, wd)
    raw = image(*tensors, pairs=[kv("general.alignment", U32, 64)], alignment=64).build()
    path = tmp_path / "paged.gguf"
    path.write_bytes(raw)
    return path, want


def _groups():
    return [[f"blk.{b}.attn_q", f"blk.{b}.ffn_down"] for b in range(BLOCKS)]


@pytest.mark.parametrize("slots", [2, 3])
def test_pager_streams_every_block_bit_identical(tmp_path, slots):
    from turbocider_amd import gguf_file, qlinear
    path, want = _model(tmp_path)
    x = activations(40, K, 7)
    xd = to_dev_bf16(x)
    with gguf_file.GGUFFile(path) as f:
        resident = qlinear.Weights()
        for g in _groups():
            for p in g:
                f.bind_projection(resident, p)
        ref = {}
        for b in range(BLOCKS):
            q = resident.project(xd, f"blk.{b}.attn_q")
            ref[b] = (from_dev_bf16(q), from_dev_bf16(resident.project(q, f"blk.{b}.ffn_down")))
        # The resident route against the oracle (block 0 and the last one).
        for b in (0, BLOCKS - 1):
            wq, bq, wd = want[b]
            wqb = oracle.bf16_to_f32(oracle.decode_matrix(wq, Q4K, N_Q, K, dtype=oracle.DTYPE_BF16))
            check(f"resident q {b}", ref[b][0], *expect(x, wqb, bq))
        with gguf_file.GGUFPager(f, _groups(), slot_count=slots) as pager:
            assert pager.slot_bytes < sum(t.bytes for t in f.tensors)
            for rnd in range(2):  # a second pass refills every slot
                seen = []
                for b, W in pager.iterate():
                    print(f"[pager] slots={slots} pass={rnd} block={b}", flush=True)
                    q = W.project(xd, f"blk.{b}.attn_q")
                    d = W.project(q, f"blk.{b}.ffn_down")
                    assert np.array_equal(from_dev_bf16(q), ref[b][0]), b
                    assert np.array_equal(from_dev_bf16(d), ref[b][1]), b
                    seen.append(b)
                assert seen == list(range(BLOCKS))
            m = pager.metrics()
            per_pass = sum(f.tensor(n).bytes for g in _groups() for p in g
                           for n in (f"{p}.weight", f"{p}.bias") if n in f._index)
            assert m["fills"] == 2 * BLOCKS and m["bytes_read"] == 2 * per_pass


def test_pager_slot_protocol_errors(tmp_path):
    from turbocider_amd import _lib, gguf_file
    path, _ = _model(tmp_path)
    with gguf_file.GGUFFile(path) as f, gguf_file.GGUFPager(f, _groups(), slot_count=2) as pager:
        t0 = pager.fill(0, 0)
        with pytest.raises(_lib.NativeError, match="slot is not vacant"):
            pager.fill(1, 0)
        with pytest.raises(_lib.NativeError, match="slot is not in use"):
            pager.retire(t0)
        W = pager.bind(t0)
        with pytest.raises(_lib.NativeError, match="slot is not ready"):
            pager.bind(t0)
        pager.retire(t0)
        del W
        t1 = pager.fill(1, 0)  # refill: the old ticket is stale
        with pytest.raises(_lib.NativeError, match="stale slot ticket"):
            pager.bind(t0)
        W = pager.bind(t1)
        pager.retire(t1)
        del W
        with pytest.raises(_lib.NativeError, match="group out of range"):
            pager.fill(BLOCKS, 1)
        with pytest.raises(_lib.NativeError, match="slot out of range"):
            pager.fill(0, 2)


def test_pager_cancel_and_changed_source(tmp_path):
    from turbocider_amd import _lib, gguf_file
    path, _ = _model(tmp_path)
    with gguf_file.GGUFFile(path) as f, gguf_file.GGUFPager(f, _groups(), slot_count=2) as pager:
        pager.cancel()
        t = pager.fill(0, 0)
        with pytest.raises(_lib.NativeCancelled, match="fill cancelled"):
            pager.bind(t)
        pager.resume()
        t = pager.fill(0, 0)  # a failed fill leaves the slot vacant
        W = pager.bind(t)
        pager.retire(t)
        del W
        # Truncate the file under the pager: the next fill's reads come up short.
        os.truncate(path, f.data_offset + 16)
        t = pager.fill(BLOCKS - 1, 1)
        with pytest.raises(_lib.NativeError, match="payload read failed or source changed"):
            pager.bind(t)


def test_pager_rejects_bad_groups(tmp_path):
    from turbocider_amd import _lib, gguf_file
    path, _ = _model(tmp_path)
    with gguf_file.GGUFFile(path) as f:
        with pytest.raises(_lib.NativeError, match="gguf_tensor_missing"):
            gguf_file.GGUFPager(f, [["blk.0.nothing"]])
        with pytest.raises(_lib.NativeError, match="no groups"):
            gguf_file.GGUFPager(f, [])
