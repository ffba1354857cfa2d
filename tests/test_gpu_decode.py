"""GPU: the device decoder is bit-exact to the reference's decoder, and the device quantizer
produces the oracle quantizer's bytes.

All calls go through the C ABI (tc_gguf_decode_device / tc_gguf_quantize_device) via the
ctypes binding in turbocider_amd.gguf.
"""
from __future__ import annotations

import random
import struct

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gguf():
    from turbocider_amd import gguf as g
    return g


def device_decode(g, raw: bytes, typ, source_rows, source_cols, row_begin=0, rows=None, column_begin=0,
                  columns=None, dtype=0, row_stride=None, column_stride=None, gather=None, fill=0xA5):
    """Same argument defaulting as oracle.decode_raw; returns (status, bytes, error)."""
    rows = source_rows if rows is None else rows
    if gather is not None:
        rows = len(gather)
    columns = source_cols - column_begin if columns is None else columns
    item = 4 if dtype == 0 else 2
    column_stride = item if column_stride is None else column_stride
    row_stride = columns * column_stride if row_stride is None else row_stride
    size = (rows - 1) * row_stride + columns * column_stride
    src = torch.tensor(list(raw), dtype=torch.uint8, device="cuda")
    dst = torch.full((size,), fill, dtype=torch.uint8, device="cuda")
    pm = g.PackedMatrix(src, typ, source_rows, source_cols)
    tgt = g.DecodeTarget(dst, g.DecodeDType(dtype), row_stride, column_stride)
    try:
        if gather is not None:
            g.decode_gather(pm, gather, column_begin, columns, tgt)
        else:
            g.decode_into(pm, g.DecodeSlice(row_begin, rows, column_begin, columns), tgt)
    except g.DecodeError as e:
        return 1, b"", str(e)
    return 0, dst.cpu().numpy().tobytes(), ""


@pytest.mark.parametrize("which", ["kquant", "other"])
def test_device_decode_matches_reference_golden(gguf, golden, other_golden, which):
    """Every golden case of the reference's decoder, K-quants and the other registered types
    (F32 / F16 / BF16 elements, Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q8_0 blocks)."""
    manifest, arrays = golden if which == "kquant" else other_golden
    keys = ("row_begin", "rows", "column_begin", "columns", "row_stride", "column_stride", "gather")
    for name, entry in sorted(manifest.items()):
        print(f"[golden] {name}", flush=True)
        raw = arrays[f"{name}__raw"].tobytes()
        kw = {k: entry[k] for k in keys if k in entry}
        for dtype in (0, 1, 2):
            status, out, err = device_decode(gguf, raw, entry["type"], entry["source_rows"], entry["source_cols"],
                                             dtype=dtype, **kw)
            assert status == entry[f"status_d{dtype}"], (name, dtype, err)
            if status == 0:
                assert out == arrays[f"{name}__d{dtype}"].tobytes(), (name, dtype)
            else:
                assert err == entry[f"error_d{dtype}"], (name, dtype, err)


def test_device_decode_random_matrices_match_oracle(gguf):
    rng = np.random.default_rng(42)
    for typ in (12, 13, 14):
        rows, cols = 37, 12 * 256
        raw = rng.integers(0, 256, size=rows * cols // 256 * oracle.BLOCK_BYTES[typ], dtype=np.uint8)
        bb = oracle.BLOCK_BYTES[typ]
        for b in range(rows * cols // 256):  # finite scales drawn like N(0, 0.02) weights would give
            off = b * bb + (208 if typ == 14 else 0)
            raw[off:off + 2] = np.frombuffer(struct.pack("<e", float(rng.uniform(-0.01, 0.01))), dtype=np.uint8)
            if typ != 14:
                raw[b * bb + 2:b * bb + 4] = np.frombuffer(struct.pack("<e", float(rng.uniform(0, 0.01))),
                                                           dtype=np.uint8)
        for dtype in (0, 2):
            print(f"[random] type={typ} dtype={dtype}", flush=True)
            want = oracle.decode_matrix(raw, typ, rows, cols, dtype=dtype)
            got = gguf.dequantize(torch.from_numpy(raw).cuda(), typ, rows, cols, gguf.DecodeDType(dtype))
            got = got.cpu().view(torch.int32 if dtype == 0 else torch.int16).numpy()
            assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), (typ, dtype)


def test_device_decode_slices_strides_and_gather(gguf):
    rng = random.Random(7)
    for typ in (12, 14):
        raw = bytes(rng.randrange(256) for _ in range(4 * 3 * oracle.BLOCK_BYTES[typ]))
        raw = bytearray(raw)
        for b in range(12):
            off = b * oracle.BLOCK_BYTES[typ] + (208 if typ == 14 else 0)
            raw[off:off + 2] = struct.pack("<e", 0.01 * (b + 1))
            if typ != 14:  # finite, small dmin too, so that every target dtype decodes
                raw[off + 2:off + 4] = struct.pack("<e", 0.005 * (b + 1))
        raw = bytes(raw)
        cases = [dict(column_begin=1, columns=700, column_stride=6, row_stride=4300),
                 dict(row_begin=1, rows=2, column_begin=255, columns=2),
                 dict(gather=[3, 3, 0, 2], column_begin=17, columns=511)]
        for kw in cases:
            for dtype in (0, 1, 2):
                print(f"[slice] type={typ} {kw} dtype={dtype}", flush=True)
                mine = device_decode(gguf, raw, typ, 4, 768, dtype=dtype, **kw)
                ref = oracle.decode_raw(raw, typ, 4, 768, dtype=dtype, fill=0xA5, **kw)
                assert mine[0] == ref[0] == 0, (typ, kw, dtype, mine[2], ref[3])
                assert mine[1] == ref[1], (typ, kw, dtype)


def test_device_decode_nonfinite_and_cancel(gguf):
    raw = bytearray(oracle.quantize(12, np.ones((1, 256), dtype=np.float32)).tobytes())
    raw[0:2] = struct.pack("<H", 0x7C00)
    status, _, err = device_decode(gguf, bytes(raw), 12, 1, 256)
    assert status == 1 and err == "nonfinite weight/scale or conversion overflow"
    src = torch.zeros(144, dtype=torch.uint8, device="cuda")
    dst = torch.full((512,), 0xA5, dtype=torch.uint8, device="cuda")
    with pytest.raises(gguf.DecodeCancelled):
        gguf.decode_into(gguf.PackedMatrix(src, 12, 1, 256), gguf.DecodeSlice(0, 1, 0, 256),
                         gguf.DecodeTarget(dst, gguf.DecodeDType.bf16, 512, 2), cancel=True)
    assert (dst.cpu() == 0xA5).all()  # nothing written


def test_device_quantizer_matches_oracle_bytes(gguf):
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    w[1, :256] = 0.0
    w[2, 256:512] = np.abs(w[2, 256:512])
    w[5, :] *= 50.0
    for typ in (12, 14):
        print(f"[quantize] type={typ}", flush=True)
        got = gguf.quantize(torch.from_numpy(w).cuda(), typ).cpu().numpy()
        assert np.array_equal(got, oracle.quantize(typ, w)), typ


OTHER_TYPES = (0, 1, 30, 2, 3, 6, 7, 8)


def other_matrix(typ, rows, cols, rng):
    """Random finite payload of a non-K type (scales / minimums small and finite)."""
    el, bb = oracle.BLOCK_ELEMENTS[typ], oracle.BLOCK_BYTES[typ]
    if typ == 0:
        return (rng.standard_normal(rows * cols).astype(np.float32) * 3).tobytes()
    if typ == 1:
        return (rng.standard_normal(rows * cols) * 3).astype(np.float16).tobytes()
    if typ == 30:
        return oracle.bf16_bits((rng.standard_normal(rows * cols) * 3).astype(np.float32)).tobytes()
    raw = rng.integers(0, 256, size=rows * cols // el * bb, dtype=np.uint8)
    for b in range(rows * cols // el):
        raw[b * bb:b * bb + 2] = np.frombuffer(struct.pack("<e", float(rng.uniform(-0.02, 0.02))), dtype=np.uint8)
        if typ in (3, 7):
            raw[b * bb + 2:b * bb + 4] = np.frombuffer(struct.pack("<e", float(rng.uniform(-0.1, 0.1))), dtype=np.uint8)
    return raw.tobytes()


@pytest.mark.parametrize("typ", OTHER_TYPES)
def test_device_decode_other_types_match_oracle(gguf, typ):
    """Random matrices of each non-K type against the oracle (pinned to the reference decoder):
    whole matrix, a slice starting and ending inside a quad / block, a strided target, a gather;
    every target dtype."""
    rng = np.random.default_rng(100 + typ)
    el = oracle.BLOCK_ELEMENTS[typ]
    rows, cols = 37, (24 * el if el > 1 else 998)
    raw = other_matrix(typ, rows, cols, rng)
    cases = [dict(), dict(column_begin=el // 2 + 3, columns=cols - el - 5), dict(column_stride=6, columns=cols - 1),
             dict(gather=[36, 0, 5, 5], column_begin=1, columns=cols - 2), dict(row_begin=30, rows=7)]
    for kw in cases:
        for dtype in (0, 1, 2):
            print(f"[other] type={typ} {kw} dtype={dtype}", flush=True)
            if "column_stride" in kw and dtype == 0:
                kw = dict(kw, column_stride=12)
            mine = device_decode(gguf, raw, typ, rows, cols, dtype=dtype, **kw)
            ref = oracle.decode_raw(raw, typ, rows, cols, dtype=dtype, fill=0xA5, **kw)
            assert mine[0] == ref[0], (typ, kw, dtype, mine[2], ref[3])
            if ref[0] == 0:
                assert mine[1] == ref[1], (typ, kw, dtype)
            else:
                assert mine[2] == ref[3], (typ, kw, dtype)


def test_device_decode_float_copy_path_errors(gguf):
    """A float source into its own dtype with a dense target is the reference's checked copy:
    a non-finite element reports 'nonfinite source float'; through another dtype (or a strided
    target) the decode path's message; F32 -> bf16 / f16 overflow is an error."""
    for typ, dtype, width, bad in ((0, 0, 4, 0x7FC00000), (1, 1, 2, 0x7C00), (30, 2, 2, 0x7F81)):
        vals = np.arange(64, dtype=np.float32) * 0.25
        raw = bytearray(vals.tobytes() if typ == 0 else vals.astype(np.float16).tobytes() if typ == 1
                        else oracle.bf16_bits(vals).tobytes())
        raw[9 * width:10 * width] = bad.to_bytes(width, "little")
        st, _, err = device_decode(gguf, bytes(raw), typ, 1, 64, dtype=dtype)
        assert st == 1 and err == "nonfinite source float", (typ, err)
        st, _, err = device_decode(gguf, bytes(raw), typ, 1, 64, dtype=dtype, column_stride=2 * width)
        assert st == 1 and err == "nonfinite weight/scale or conversion overflow", (typ, err)
    big = struct.pack("<I", 0x7F7FFFFF) * 8
    assert device_decode(gguf, big, 0, 1, 8, dtype=2)[::2] == (1, "BF16 conversion overflow")
    assert device_decode(gguf, big, 0, 1, 8, dtype=1)[::2] == (1, "FP16 conversion overflow")
