"""CPU: the host-pointer decode (tc_gguf_decode_host, the product's own CPU decoder) against the
reference decoder's golden vectors, through the C ABI.

Every golden case (tests/golden/, written by the reference's compiled gguf_decode.cpp) is decoded
into a guard-filled target for each target dtype: bytes, status, message and the receipt's first
four fields must equal the reference's. Also: random rows of every type against the oracle,
cancellation before any write, and the geometry errors in the reference's order. No GPU.
"""
from __future__ import annotations

import hashlib
import struct

import numpy as np
import pytest

from oracle import oracle
from turbocider_amd import gguf

KEYS = ("row_begin", "rows", "column_begin", "columns", "row_stride", "column_stride", "gather")


def host_decode(raw: bytes, typ, source_rows, source_cols, row_begin=0, rows=None, column_begin=0, columns=None,
                dtype=0, row_stride=None, column_stride=None, gather=None, fill=0xA5, cancel=False):
    """Same argument defaulting as oracle.decode_raw; returns (status, target bytes, receipt, error)."""
    rows = len(gather) if gather is not None else (source_rows if rows is None else rows)
    columns = source_cols - column_begin if columns is None else columns
    item = 4 if dtype == 0 else 2
    column_stride = item if column_stride is None else column_stride
    row_stride = columns * column_stride if row_stride is None else row_stride
    size = (rows - 1) * row_stride + columns * column_stride
    src = np.frombuffer(raw, dtype=np.uint8).copy()
    dst = np.full(size, fill, dtype=np.uint8)
    pm = gguf.PackedMatrix(src, typ, source_rows, source_cols)
    tgt = gguf.DecodeTarget(dst, gguf.DecodeDType(dtype), row_stride, column_stride)
    try:
        if gather is not None:
            rc = gguf.decode_cpu_gather(pm, gather, column_begin, columns, tgt, cancel=cancel)
        else:
            rc = gguf.decode_cpu_into(pm, gguf.DecodeSlice(row_begin, rows, column_begin, columns), tgt, cancel=cancel)
    except gguf.DecodeCancelled as e:
        return 2, dst.tobytes(), None, str(e)
    except gguf.DecodeError as e:
        return 1, dst.tobytes(), None, str(e)
    return 0, dst.tobytes(), rc, ""


@pytest.mark.parametrize("which", ["kquant", "other"])
def test_host_decode_matches_reference_golden(golden, other_golden, which):
    manifest, arrays = golden if which == "kquant" else other_golden
    for name, entry in sorted(manifest.items()):
        raw = arrays[f"{name}__raw"].tobytes()
        kw = {k: entry[k] for k in KEYS if k in entry}
        for dtype in (0, 1, 2):
            status, out, rc, err = host_decode(raw, entry["type"], entry["source_rows"], entry["source_cols"],
                                               dtype=dtype, **kw)
            assert status == entry[f"status_d{dtype}"], (name, dtype, err)
            if status == 0:
                assert out == arrays[f"{name}__d{dtype}"].tobytes(), (name, dtype)
                assert hashlib.sha256(out).hexdigest() == entry[f"sha256_d{dtype}"], (name, dtype)
                want_rc = entry[f"receipt_d{dtype}"]
                got_rc = [rc.source_bytes_processed, rc.elements_written, rc.bytes_written, rc.scratch_bytes]
                assert got_rc == want_rc, (name, dtype, got_rc, want_rc)
                assert rc.scratch_bytes == 1024 and rc.simd_blocks == 0
            else:
                assert err == entry[f"error_d{dtype}"], (name, dtype, err)


def _finite_blocks(rng, typ, rows, cols):
    bb, el = oracle.BLOCK_BYTES[typ], oracle.BLOCK_ELEMENTS[typ]
    if el == 1:
        w = (rng.standard_normal(rows * cols) * 0.5).astype(np.float32)
        return (w if typ == 0 else w.astype(np.float16) if typ == 1 else oracle.bf16_bits(w)).view(np.uint8)
    raw = rng.integers(0, 256, size=rows * cols // el * bb, dtype=np.uint8)
    blocks = raw.reshape(-1, bb)
    scale_at = 208 if typ == 14 else 0
    for i in range(len(blocks)):
        blocks[i, scale_at:scale_at + 2] = np.frombuffer(struct.pack("<e", float(rng.uniform(-0.02, 0.02))), np.uint8)
        if typ in (3, 7, 12, 13):
            blocks[i, 2:4] = np.frombuffer(struct.pack("<e", float(rng.uniform(-0.01, 0.01))), np.uint8)
    return raw


@pytest.mark.parametrize("typ", sorted(oracle.BLOCK_BYTES))
def test_host_decode_random_rows_match_oracle(typ):
    """Random finite rows of every registered type, every dtype, a strided column slice."""
    rng = np.random.default_rng(300 + typ)
    rows, cols = 5, 512
    raw = _finite_blocks(rng, typ, rows, cols).tobytes()
    for dtype in (0, 1, 2):
        for kw in ({}, dict(row_begin=1, rows=3, column_begin=7, columns=300, column_stride=6, row_stride=2000),
                   dict(gather=[4, 0, 4], column_begin=32, columns=256)):
            mine = host_decode(raw, typ, rows, cols, dtype=dtype, **kw)
            ref = oracle.decode_raw(raw, typ, rows, cols, dtype=dtype, fill=0xA5, **kw)
            assert mine[0] == ref[0], (typ, dtype, kw, mine[3], ref[3])
            if ref[0] == 0:
                assert mine[1] == ref[1], (typ, dtype, kw)
            else:
                assert mine[3] == ref[3], (typ, dtype, kw)


def test_host_decode_cancel_and_errors():
    raw = oracle.quantize(12, np.ones((2, 256), dtype=np.float32)).tobytes()
    status, out, _, err = host_decode(raw, 12, 2, 256, cancel=True)
    assert status == 2 and err == "gguf_decode_cancelled"
    assert set(out) == {0xA5}  # pre-set cancellation writes nothing
    # Geometry errors (gguf_decode.cpp:160-183 order).
    assert host_decode(raw, 99, 2, 256)[3] == "gguf_decode: unsupported tensor type"
    assert host_decode(raw, 12, 2, 300)[3] == "invalid source geometry"
    assert host_decode(raw, 12, 2, 256, row_begin=1, rows=2)[3] == "row slice out of bounds"
    assert host_decode(raw[:-1], 12, 2, 256)[3] == "packed source too short"
    assert host_decode(raw, 12, 2, 256, column_stride=2, dtype=0)[3] == "invalid/overlapping column stride"
    assert host_decode(raw, 12, 2, 256, row_stride=100, dtype=2)[3] == "invalid/overlapping row stride"
    assert host_decode(raw, 12, 2, 256, gather=[0, 2])[3] == "gather row out of bounds"
    bad = bytearray(raw)
    bad[144:146] = struct.pack("<H", 0x7E00)  # row 1: NaN d
    status, _, _, err = host_decode(bytes(bad), 12, 2, 256)
    assert status == 1 and err == "nonfinite weight/scale or conversion overflow"


def test_host_decode_threads_split_rows():
    """Reentrant: two threads decoding disjoint row ranges into one target give the whole
    matrix."""
    from concurrent.futures import ThreadPoolExecutor
    rng = np.random.default_rng(5)
    rows, cols = 64, 1024
    raw = _finite_blocks(rng, 14, rows, cols)
    out = np.zeros((rows, cols), dtype=np.uint16)

    def part(r0):
        tgt = gguf.DecodeTarget(out[r0:r0 + 32], gguf.DecodeDType.bf16, cols * 2, 2)
        return gguf.decode_cpu_into(gguf.PackedMatrix(raw, 14, rows, cols), gguf.DecodeSlice(r0, 32, 0, cols), tgt)
    with ThreadPoolExecutor(2) as pool:
        list(pool.map(part, (0, 32)))
    assert np.array_equal(out, oracle.decode_matrix(raw, 14, rows, cols, dtype=oracle.DTYPE_BF16))
