"""CPU: pin the C oracle's decode against the reference's own decoder.

Pins, in order of strength:
1. golden vectors written by the reference's gguf_decode.cpp compiled unmodified
   (tests/golden/make_golden.py): every case, every target dtype, status, bytes, receipt;
2. when oracle/_ref is built here, fresh random blocks through both decoders;
3. the fp16/bf16 conversion KATs of tests/native/test_gguf_execution.py:176-198
   (exhaustive finite fp16 round trip against IEEE half from numpy, RNE ties);
4. an exact-rational closed form of the K-quant expressions (float64 is exact for
   d*sc*q - dmin*m, rounded once to float32), from a numpy layout restatement;
5. invariants: slices / gathers equal sub-blocks of the full decode, bf16 = RNE(f32),
   guard bytes untouched, rejected geometry.
"""
from __future__ import annotations

import random
import struct

import numpy as np
import pytest

from oracle import oracle

TYPES = (12, 13, 14)
OTHER_TYPES = (0, 1, 30, 2, 3, 6, 7, 8)  # F32, F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0


def _call_kwargs(entry):
    keys = ("row_begin", "rows", "column_begin", "columns", "row_stride", "column_stride", "gather")
    return {k: entry[k] for k in keys if k in entry}


@pytest.mark.parametrize("which", ["kquant", "other"])
def test_oracle_matches_reference_golden(golden, other_golden, which):
    manifest, arrays = golden if which == "kquant" else other_golden
    checked = 0
    for name, entry in manifest.items():
        raw = arrays[f"{name}__raw"].tobytes()
        for dtype in (0, 1, 2):
            status, out, stats, err = oracle.decode_raw(raw, entry["type"], entry["source_rows"],
                                                        entry["source_cols"], dtype=dtype, fill=0xA5,
                                                        **_call_kwargs(entry))
            assert status == entry[f"status_d{dtype}"], (name, dtype, err)
            if status == 0:
                assert out == arrays[f"{name}__d{dtype}"].tobytes(), (name, dtype)
                assert stats[:4] == entry[f"receipt_d{dtype}"], (name, dtype)
            else:
                assert err == entry[f"error_d{dtype}"], (name, dtype)
            checked += 1
    assert checked == 3 * len(manifest) and len(manifest) >= 50
    assert {e["type"] for e in manifest.values()} == ({12, 13, 14} if which == "kquant" else set(OTHER_TYPES))


def random_block(typ, rng):
    size = oracle.BLOCK_BYTES[typ]
    data = bytearray(rng.randbytes(size))
    off = 208 if typ == 14 else 0
    data[off:off + 2] = struct.pack("<e", rng.choice([0.0, -0.0, 2 ** -24, -0.125, 0.03125, 1.5, 0.0017, -3.0]))
    if typ in (12, 13):
        data[2:4] = struct.pack("<e", rng.choice([0.0, -0.5, 0.25, 2 ** -24, 0.001]))
    return bytes(data)


def test_oracle_matches_reference_decoder_random(ref_decoder):
    rng = random.Random(6409)
    for typ in TYPES:
        for trial in range(24):
            raw = b"".join(random_block(typ, rng) for _ in range(12))
            for dtype in (0, 1, 2):
                mine = oracle.decode_raw(raw, typ, 3, 1024, dtype=dtype)
                ref = oracle.decode_raw(raw, typ, 3, 1024, dtype=dtype, use_ref=True)
                assert mine[0] == ref[0] and (mine[0] or mine[1] == ref[1]), (typ, trial, dtype)


def test_fp16_exhaustive_round_trip():
    bits = np.arange(65536, dtype=np.uint32)
    finite = bits[(bits & 0x7C00) != 0x7C00]
    assert finite.size == 63488
    expected = finite.astype(np.uint16).view(np.float16).astype(np.float32)
    L = oracle.lib()
    got = np.array([L.oracle_fp16_to_float(int(b)) for b in finite], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))
    for b, v in zip(finite[::97], got[::97]):
        status, h = oracle.round_fp16(float(v))
        assert status == 0 and h == b


def test_rounding_ties_subnormals_and_overflow():
    for value in [0., -0., 2 ** -25, -2 ** -25, 3 * 2 ** -25, 1 + 2 ** -11, 1 + 3 * 2 ** -11, 65504., -65504.]:
        status, h = oracle.round_fp16(value)
        assert status == 0 and h == struct.unpack("<H", struct.pack("<e", value))[0], value
    for value in [65520., -65520., float("inf"), float("nan")]:
        assert oracle.round_fp16(value)[0] != 0
    for bits in [0x3F808000, 0x3F818000, 0xBF808000, 1, 0x80000001, 0x7F7FFFFF]:
        value = struct.unpack("<f", struct.pack("<I", bits))[0]
        status, h = oracle.round_bf16(value)
        expected = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
        assert (status == 0) == ((expected & 0x7F80) != 0x7F80)
        if status == 0:
            assert h == expected


# ---------------------------------------------------------------------------------------
# exact-rational closed form (independent numpy layout restatement)
# ---------------------------------------------------------------------------------------
def _k4_scale_min(s: np.ndarray, g: int):
    if g < 4:
        return s[g] & 63, s[g + 4] & 63
    return (s[g + 4] & 15) | ((s[g - 4] >> 6) << 4), (s[g + 4] >> 4) | ((s[g] >> 6) << 4)


def closed_form_block(typ: int, blk: bytes) -> np.ndarray:
    b = np.frombuffer(blk, dtype=np.uint8).astype(np.int64)
    out = np.empty(256, dtype=np.float64)
    if typ in (12, 13):
        d = float(np.frombuffer(blk[0:2], dtype=np.float16)[0])
        dmin = float(np.frombuffer(blk[2:4], dtype=np.float16)[0])
        qs = b[48:176] if typ == 13 else b[16:144]
        for g in range(8):
            sc, m = _k4_scale_min(b[4:16], g)
            q = (qs[32 * (g // 2): 32 * (g // 2) + 32] >> (4 * (g % 2))) & 15
            if typ == 13:
                q = q + (((b[16:48] >> g) & 1) << 4)
            out[32 * g: 32 * g + 32] = d * sc * q - dmin * m
    else:
        d = float(np.frombuffer(blk[208:210], dtype=np.float16)[0])
        sc = b[192:208].astype(np.int8).astype(np.int64)
        for i in range(256):
            h, g, j = i // 128, (i % 128) // 32, i % 32
            lo = (b[64 * h + 32 * (g % 2) + j] >> (4 * (g // 2))) & 15
            hi = (b[128 + 32 * h + j] >> (2 * g)) & 3
            out[i] = d * sc[8 * h + 2 * g + j // 16] * ((lo | (hi << 4)) - 32)
    return out.astype(np.float32)  # one RNE rounding of the exact value


def test_closed_form_matches_oracle():
    rng = random.Random(1234)
    for typ in TYPES:
        for _ in range(40):
            blk = random_block(typ, rng)
            status, out, _, _ = oracle.decode_raw(blk, typ, 1, 256, dtype=0)
            assert status == 0
            got = np.frombuffer(out, dtype=np.float32)
            want = closed_form_block(typ, blk)
            # compare bit patterns, but treat +0 / -0 alike (exact zero of the difference)
            g, w = got.view(np.uint32), want.view(np.uint32)
            zero = (g & 0x7FFFFFFF) == 0
            assert np.array_equal(zero, (w & 0x7FFFFFFF) == 0)
            assert np.array_equal(g[~zero], w[~zero]), typ


def test_closed_form_catches_planted_mistake():
    """The closed form is sensitive: a transposed nibble choice (high for even sub-blocks)
    planted into the restatement must disagree with the oracle."""
    rng = random.Random(99)
    blk = bytearray(random_block(12, rng))
    blk[0:2] = struct.pack("<e", 0.5)
    blk[2:4] = struct.pack("<e", 0.25)
    good = closed_form_block(12, bytes(blk))
    swapped = bytearray(blk)
    swapped[16:144] = bytes(((x >> 4) | ((x & 15) << 4)) for x in blk[16:144])
    bad = closed_form_block(12, bytes(swapped))
    _, out, _, _ = oracle.decode_raw(bytes(blk), 12, 1, 256, dtype=0)
    got = np.frombuffer(out, dtype=np.float32)
    assert np.array_equal(got, good) and not np.array_equal(got, bad)


def test_slices_gather_and_bf16_invariants():
    rng = random.Random(20260930)
    for typ in TYPES:
        cols = 3 * 256
        raw = b"".join(random_block(typ, rng) for _ in range(9))
        status, full, _, _ = oracle.decode_raw(raw, typ, 3, cols, dtype=0)
        assert status == 0
        full = np.frombuffer(full, dtype=np.float32).reshape(3, cols)
        for begin, count in [(0, cols), (1, cols - 2), (255, 258), (300, 1)]:
            st, out, _, _ = oracle.decode_raw(raw, typ, 3, cols, column_begin=begin, columns=count, dtype=0,
                                              column_stride=8, row_stride=count * 8 + 8, fill=0xA5)
            assert st == 0
            buf = np.frombuffer(out, dtype=np.uint8)
            for r in range(3):
                row = buf[r * (count * 8 + 8):]
                vals = np.frombuffer(row[: count * 8].tobytes(), dtype=np.float32)[::2]
                assert np.array_equal(vals.view(np.uint32), full[r, begin:begin + count].view(np.uint32))
                pad = row[: count * 8].reshape(count, 8)[:, 4:]
                assert (pad == 0xA5).all()
            st, out2, _, _ = oracle.decode_raw(raw, typ, 3, cols, column_begin=begin, columns=count, dtype=2)
            bf = np.frombuffer(out2, dtype=np.uint16).reshape(3, count)
            assert np.array_equal(bf, oracle.bf16_bits(full[:, begin:begin + count]))
        st, g, _, _ = oracle.decode_raw(raw, typ, 3, cols, gather=[2, 0, 2], dtype=0)
        assert st == 0
        g = np.frombuffer(g, dtype=np.float32).reshape(3, cols)
        assert np.array_equal(g, full[[2, 0, 2]])


def test_rejected_geometry_and_cancellation():
    raw = random_block(12, random.Random(5))
    bad = [dict(source_columns=255), dict(source_rows=2), dict(rows=2), dict(column_begin=250, columns=7),
           dict(dtype=99), dict(column_stride=0), dict(row_stride=1), dict(target_size=1), dict(gather=[1]),
           dict(cancel=True)]
    for override in bad:
        args = dict(raw=raw, typ=12, source_rows=1, source_columns=256)
        args.update(override)
        status = oracle.decode_raw(**args)[0]
        assert status != 0, override
    assert oracle.decode_raw(raw, 12, 1, 256, cancel=True)[0] == 2
    for scale in (float("inf"), float("nan")):
        blk = bytearray(raw)
        blk[0:2] = struct.pack("<e", scale)
        assert oracle.decode_raw(bytes(blk), 12, 1, 256)[0] == 1


def test_quantizer_properties():
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((16, 1024)) * 0.02).astype(np.float32)
    w[3, :256] = 0.0                       # an all-zero super-block
    w[4, 256:512] = np.abs(w[4, 256:512])  # a non-negative one (min clamps to 0)
    for typ in (12, 14):
        blocks = oracle.quantize(typ, w)
        assert np.array_equal(blocks, oracle.quantize(typ, w))  # deterministic
        dec = oracle.decode_matrix(blocks, typ, 16, 1024)
        assert np.isfinite(dec).all()
        err = np.abs(dec - w).reshape(16, 4, 256)
        span = (w.reshape(16, 4, 256).max(-1) - np.minimum(w.reshape(16, 4, 256).min(-1), 0))
        # codes are re-derived from the stored (rounded) sub-scales: within one code step
        # of the sub-block range (Q4_K: 15 steps, Q6_K: 31..32 steps) plus scale rounding
        bound = span / (15.0 if typ == 12 else 24.0)
        assert (err.max(-1) <= bound + 1e-6).all(), typ
        rel = np.linalg.norm(dec - w) / np.linalg.norm(w)
        assert rel < (0.12 if typ == 12 else 0.03), (typ, rel)
        assert np.all(dec[3, :256] == 0)
        if typ == 12:  # dmin of the all-zero and the non-negative super-blocks is +0, not -0
            for row, blk in ((3, 0), (4, 1)):
                off = (row * 4 + blk) * 144
                assert blocks[off + 2] == 0 and blocks[off + 3] == 0


# ---------------------------------------------------------------------------------------
# The other registered types: F32 / F16 / BF16 elements and the legacy 32-weight blocks
# (gguf_decode.cpp:56-76, 119-158).
# ---------------------------------------------------------------------------------------
SCALES = [0.0, -0.0, 2 ** -24, -0.125, 0.03125, 1.5, 0.0017, -3.0, 65504.0]


def random_other_block(typ, rng, nonfinite=False):
    """One block of `typ`: random payload with scale (and minimum) fp16 values from the
    reference tests' choices; float types get finite random values of their width."""
    if typ == 0:
        v = rng.choice([0.0, -0.0, 1.5, -3.25e-3, 6.1e4, 1e-40, 3.0e38, -1.7e38]) * rng.choice([1, -1])
        if nonfinite:
            v = rng.choice([float("inf"), float("nan")])
        return struct.pack("<f", v)
    if typ in (1, 30):
        while True:
            bits = rng.randrange(65536)
            finite = (bits & (0x7C00 if typ == 1 else 0x7F80)) != (0x7C00 if typ == 1 else 0x7F80)
            if finite != nonfinite:
                return struct.pack("<H", bits)
    size = oracle.BLOCK_BYTES[typ]
    data = bytearray(rng.randbytes(size))
    data[0:2] = struct.pack("<e", float("inf") if nonfinite else rng.choice(SCALES))
    if typ in (3, 7):
        data[2:4] = struct.pack("<e", rng.choice([0.0, -0.5, 0.25, 2 ** -24, 0.001, -60000.0]))
    return bytes(data)


@pytest.mark.parametrize("typ", OTHER_TYPES)
def test_other_types_match_reference_decoder(ref_decoder, typ):
    """Random rows through both decoders: every target dtype, dense (the same-dtype copy path for
    float sources) and strided targets, column slices, gathers, status and error text."""
    rng = random.Random(1000 + typ)
    el = oracle.BLOCK_ELEMENTS[typ]
    cols = 4 * el if el > 1 else 96
    per_row = cols // el
    for trial in range(16):
        bad = trial % 5 == 4
        blocks = [random_other_block(typ, rng, nonfinite=bad and i == 5) for i in range(3 * per_row)]
        raw = b"".join(blocks)
        for dtype in (0, 1, 2):
            item = 4 if dtype == 0 else 2
            for kw in ({}, dict(column_begin=el // 2 + 1, columns=cols - el), dict(column_stride=2 * item),
                       dict(gather=[2, 0, 2])):
                mine = oracle.decode_raw(raw, typ, 3, cols, dtype=dtype, **kw)
                ref = oracle.decode_raw(raw, typ, 3, cols, dtype=dtype, use_ref=True, **kw)
                assert mine[0] == ref[0], (typ, trial, dtype, kw, mine[3], ref[3])
                if mine[0] == 0:
                    assert mine[1] == ref[1] and mine[2][:4] == ref[2][:4], (typ, trial, dtype, kw)
                else:
                    assert mine[3] == ref[3], (typ, trial, dtype, kw)


def test_other_types_closed_forms():
    """The legacy block expressions restated from the layout with numpy (float64 is exact for
    code * scale [+ minimum] before the single float32 rounding), a planted mistake fails."""
    rng = random.Random(77)

    def expect(typ, blk, swap=False):
        b = np.frombuffer(blk, dtype=np.uint8)
        d = float(np.frombuffer(blk[0:2], dtype=np.float16)[0])
        if typ == 8:
            return (np.frombuffer(blk[2:34], dtype=np.int8).astype(np.float64) * d).astype(np.float32)
        affine, five = typ in (3, 7), typ in (6, 7)
        m = float(np.frombuffer(blk[2:4], dtype=np.float16)[0]) if affine else 0.0
        off = 4 if affine else 2
        high = int.from_bytes(blk[off:off + 4], "little") if five else 0
        low = b[off + (4 if five else 0):][:16].astype(np.int64)
        lo, hi = low & 15, low >> 4
        if swap:
            lo, hi = hi, lo
        if five:
            lo = lo | (((high >> np.arange(16)) & 1) << 4)
            hi = hi | (((high >> (np.arange(16) + 16)) & 1) << 4)
        codes = np.concatenate([lo, hi]).astype(np.float64)
        if not affine:
            codes -= 16 if five else 8
            return (codes * d).astype(np.float32)  # no "+ 0.0": it would turn -0 into +0
        return (codes * d + m).astype(np.float32)

    for typ in (2, 3, 6, 7, 8):
        for _ in range(40):
            blk = random_other_block(typ, rng)
            st, out, _, _ = oracle.decode_raw(blk, typ, 1, 32, dtype=0)
            assert st == 0
            got = np.frombuffer(out, dtype=np.float32)
            assert np.array_equal(got.view(np.uint32), expect(typ, blk).view(np.uint32)), typ
        if typ != 8:
            blk = bytearray(random_other_block(typ, rng))
            blk[0:2] = struct.pack("<e", 1.0)
            blk[len(blk) - 16:] = bytes(range(1, 17))
            st, out, _, _ = oracle.decode_raw(bytes(blk), typ, 1, 32, dtype=0)
            got = np.frombuffer(out, dtype=np.float32)
            assert not np.array_equal(got, expect(typ, bytes(blk), swap=True)), typ


def test_other_types_copy_path_and_errors():
    """F32 -> f32, F16 -> f16, BF16 -> bf16 with a dense target is a checked byte copy
    (gguf_decode.cpp:119-158): any finite payload comes back bit for bit, a non-finite one is
    'nonfinite source float'; through another dtype the decode path's messages apply."""
    rng = np.random.default_rng(3)
    for typ, dtype, width, mask in ((0, 0, 4, 0x7F800000), (1, 1, 2, 0x7C00), (30, 2, 2, 0x7F80)):
        bits = rng.integers(0, 2 ** (8 * width), 512, dtype=np.uint64).astype(np.uint32 if width == 4 else np.uint16)
        bits = bits[(bits & mask) != mask][:256]
        raw = bits.tobytes()
        st, out, stats, _ = oracle.decode_raw(raw, typ, 1, 256, dtype=dtype)
        assert st == 0 and out == raw and stats[:3] == [256 * width, 256, 256 * width]
        bad = bytearray(raw)
        bad[7 * width:8 * width] = (mask | 1).to_bytes(width, "little")
        st, _, _, err = oracle.decode_raw(bytes(bad), typ, 1, 256, dtype=dtype)
        assert st == 1 and err == "nonfinite source float"
        other = 0 if dtype != 0 else 2
        st, _, _, err = oracle.decode_raw(bytes(bad), typ, 1, 256, dtype=other)
        assert st == 1 and err == "nonfinite weight/scale or conversion overflow"
    big = struct.pack("<I", 0x7F7FFFFF) * 32  # FLT_MAX: rounds to bf16 infinity
    assert oracle.decode_raw(big, 0, 1, 32, dtype=2)[::3] == (1, "BF16 conversion overflow")
    assert oracle.decode_raw(big, 0, 1, 32, dtype=1)[::3] == (1, "FP16 conversion overflow")
    assert oracle.decode_raw(struct.pack("<f", 3.38e38) * 32, 0, 1, 32, dtype=2)[0] == 0
