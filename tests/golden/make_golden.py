"""Write the decode golden vectors with the reference's own decoder.

Runs only where /root/reference exists: it compiles native/core/gguf_decode.cpp from where it
lies (``make -C oracle ref`` -> oracle/_ref/libggufref.so) and decodes the block sets below
through ``decode_cpu_into`` / ``decode_cpu_gather``. The committed output,
``tests/golden/kquant_golden.npz`` (+ ``kquant_golden.json`` with SHA-256 digests), is
data only: input block bytes, call parameters, status codes and output bytes.

Block sets (value choices follow the reference's own tests):
* ``rand_*``: random bytes with master scales d in {0, -0, 2^-24, -0.125, 0.03125, 1.5} and
  dmin in {0, -0.5, 0.25, 2^-24} (tests/native/test_gguf_execution.py:56-63).
* ``edge_*``: byte pattern (i*73 + b*17 + 19) & 255 with d in {0, -0, 2^-24, 0.03125, -0.03125,
  65504, -65504} and dmin -0.015625 (tests/native/gguf_decode_safety_test.cpp:64-79).
* ``quant_*``: N(0, 0.02) weights through this repo's own quantizer (oracle.quantize).
* ``nonfinite_*``: an inf / nan master scale (gguf_decode_safety_test.cpp:118-125).
* ``slice_*``: column slices and strided targets (test_gguf_execution.py:270-288) and a
  duplicate/order-preserving gather (:258-262).

A second set (``other_golden.npz`` / ``.json``, ``main_other``) covers the F32 / F16 / BF16
elements and the legacy Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q8_0 blocks the reference decoder also
handles (gguf_decode.cpp:56-76, 119-158).

Usage:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import random
import struct
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent
ELEMENTS = 256


def block(typ: int, rng: random.Random) -> bytes:
    size = oracle.BLOCK_BYTES[typ]
    data = bytearray(rng.randbytes(size))
    offset = 208 if typ == oracle.TYPE_Q6_K else 0
    data[offset:offset + 2] = struct.pack("<e", rng.choice([0.0, -0.0, 2 ** -24, -0.125, 0.03125, 1.5]))
    if typ in (oracle.TYPE_Q4_K, oracle.TYPE_Q5_K):
        data[2:4] = struct.pack("<e", rng.choice([0.0, -0.5, 0.25, 2 ** -24]))
    return bytes(data)


def edge_blocks(typ: int, scale: float, count: int) -> bytes:
    size = oracle.BLOCK_BYTES[typ]
    out = bytearray()
    for b in range(count):
        p = bytearray(((i * 73 + b * 17 + 19) & 255) for i in range(size))
        _, bits = oracle.round_fp16(scale)
        off = 208 if typ == oracle.TYPE_Q6_K else 0
        p[off:off + 2] = struct.pack("<H", bits)
        if typ in (oracle.TYPE_Q4_K, oracle.TYPE_Q5_K):
            _, mbits = oracle.round_fp16(-0.015625)
            p[2:4] = struct.pack("<H", mbits)
        out += p
    return bytes(out)


def main() -> None:
    oracle.build(ref=True)
    if oracle.ref_lib() is None:
        raise SystemExit("reference decoder not available (needs /root/reference)")
    rng = random.Random(20261201)
    arrays: dict[str, np.ndarray] = {}
    manifest: dict[str, dict] = {}

    def record(name, raw, typ, source_rows, source_cols, **kw):
        entry = {"type": typ, "source_rows": source_rows, "source_cols": source_cols,
                 **{k: v for k, v in kw.items() if k != "gather"}}
        if "gather" in kw:
            entry["gather"] = list(kw["gather"])
        arrays[f"{name}__raw"] = np.frombuffer(raw, dtype=np.uint8).copy()
        for dtype in (0, 1, 2):
            status, out, stats, err = oracle.decode_raw(raw, typ, source_rows, source_cols, dtype=dtype, use_ref=True,
                                                        fill=0xA5, **kw)
            key = f"{name}__d{dtype}"
            arrays[key] = np.frombuffer(out, dtype=np.uint8).copy()
            entry[f"status_d{dtype}"] = status
            entry[f"error_d{dtype}"] = err if status else ""
            entry[f"receipt_d{dtype}"] = stats[:4] if status == 0 else []
            entry[f"sha256_d{dtype}"] = hashlib.sha256(out).hexdigest()
        manifest[name] = entry

    for typ, tag in ((12, "q4k"), (13, "q5k"), (14, "q6k")):
        rows, blocks_per_row = 3, 8
        raw = b"".join(block(typ, rng) for _ in range(rows * blocks_per_row))
        record(f"rand_{tag}", raw, typ, rows, blocks_per_row * ELEMENTS)
        for i, scale in enumerate([0.0, -0.0, 2 ** -24, 0.03125, -0.03125, 65504.0, -65504.0]):
            record(f"edge_{tag}_{i}", edge_blocks(typ, scale, 4), typ, 2, 2 * ELEMENTS)
        for j, bad in enumerate([0x7C00, 0x7E00]):
            raw = bytearray(edge_blocks(typ, 1.0, 2))
            off = 208 if typ == 14 else 0
            raw[off:off + 2] = struct.pack("<H", bad)
            record(f"nonfinite_{tag}_{j}", bytes(raw), typ, 1, 2 * ELEMENTS)
            if typ != 14:
                raw = bytearray(edge_blocks(typ, 1.0, 2))
                off2 = oracle.BLOCK_BYTES[typ] + 2  # dmin of the second block
                raw[off2:off2 + 2] = struct.pack("<H", bad)
                record(f"nonfinite_min_{tag}_{j}", bytes(raw), typ, 1, 2 * ELEMENTS)
        cols = 3 * ELEMENTS
        raw = b"".join(block(typ, rng) for _ in range(3 * 3))
        for s, (begin, count) in enumerate([(0, cols), (1, cols - 2), (ELEMENTS - 1, ELEMENTS + 2)]):
            record(f"slice_{tag}_{s}", raw, typ, 3, cols, column_begin=begin, columns=count, column_stride=8,
                   row_stride=count * 8 + 8)
        record(f"rows_{tag}", raw, typ, 3, cols, row_begin=1, rows=2)
        record(f"gather_{tag}", raw, typ, 3, cols, gather=[2, 0, 2], column_begin=5, columns=300)

    wrng = np.random.default_rng(0)
    for typ, tag in ((12, "q4k"), (14, "q6k")):
        w = (wrng.standard_normal((8, 1024)) * 0.02).astype(np.float32)
        raw = oracle.quantize(typ, w).tobytes()
        arrays[f"quant_{tag}__w"] = w
        record(f"quant_{tag}", raw, typ, 8, 1024)

    np.savez_compressed(OUT / "kquant_golden.npz", **arrays)
    (OUT / "kquant_golden.json").write_text(json.dumps(manifest, indent=1, sort_keys=True) + "\n")
    print(f"wrote {len(manifest)} cases, {sum(a.nbytes for a in arrays.values())} bytes uncompressed")


OTHER_TAGS = {0: "f32", 1: "f16", 30: "bf16", 2: "q4_0", 3: "q4_1", 6: "q5_0", 7: "q5_1", 8: "q8_0"}


def other_block(typ: int, rng: random.Random) -> bytes:
    """Random block of a non-K type: scales (and minimums) from the reference tests' choices."""
    if typ == 0:
        return struct.pack("<f", rng.choice([0.0, -0.0, 1.5, -3.25e-3, 6.1e4, 1e-40, 3.0e38, -2.5]))
    if typ in (1, 30):
        mask = 0x7C00 if typ == 1 else 0x7F80
        while True:
            bits = rng.randrange(65536)
            if bits & mask != mask:
                return struct.pack("<H", bits)
    data = bytearray(rng.randbytes(oracle.BLOCK_BYTES[typ]))
    data[0:2] = struct.pack("<e", rng.choice([0.0, -0.0, 2 ** -24, -0.125, 0.03125, 1.5, 65504.0]))
    if typ in (3, 7):
        data[2:4] = struct.pack("<e", rng.choice([0.0, -0.5, 0.25, 2 ** -24, -60000.0]))
    return bytes(data)


def main_other() -> None:
    """Golden vectors of the F32 / F16 / BF16 and legacy 32-weight block types
    (other_golden.npz / .json): random rows, non-finite scales and elements, conversion
    overflow, slices with strided targets, row ranges and a gather."""
    rng = random.Random(20261202)
    arrays: dict[str, np.ndarray] = {}
    manifest: dict[str, dict] = {}

    def record(name, raw, typ, source_rows, source_cols, **kw):
        entry = {"type": typ, "source_rows": source_rows, "source_cols": source_cols,
                 **{k: v for k, v in kw.items() if k != "gather"}}
        if "gather" in kw:
            entry["gather"] = list(kw["gather"])
        arrays[f"{name}__raw"] = np.frombuffer(raw, dtype=np.uint8).copy()
        for dtype in (0, 1, 2):
            status, out, stats, err = oracle.decode_raw(raw, typ, source_rows, source_cols, dtype=dtype, use_ref=True,
                                                        fill=0xA5, **kw)
            arrays[f"{name}__d{dtype}"] = np.frombuffer(out, dtype=np.uint8).copy()
            entry[f"status_d{dtype}"] = status
            entry[f"error_d{dtype}"] = err if status else ""
            entry[f"receipt_d{dtype}"] = stats[:4] if status == 0 else []
            entry[f"sha256_d{dtype}"] = hashlib.sha256(out).hexdigest()
        manifest[name] = entry

    for typ, tag in OTHER_TAGS.items():
        el = oracle.BLOCK_ELEMENTS[typ]
        cols = 4 * el if el > 1 else 96
        per_row = cols // el
        raw = b"".join(other_block(typ, rng) for _ in range(3 * per_row))
        record(f"rand_{tag}", raw, typ, 3, cols)
        for s, (begin, count) in enumerate([(1, cols - 2), (el // 2 + 3, el + 5)]):
            record(f"slice_{tag}_{s}", raw, typ, 3, cols, column_begin=begin, columns=count, column_stride=8,
                   row_stride=count * 8 + 8)
        record(f"rows_{tag}", raw, typ, 3, cols, row_begin=1, rows=2)
        record(f"gather_{tag}", raw, typ, 3, cols, gather=[2, 0, 2], column_begin=3, columns=cols - 7)
        for j, bad in enumerate([0x7C00, 0x7E00]):
            blocks = [bytearray(other_block(typ, rng)) for _ in range(per_row)]
            if typ == 0:
                blocks[per_row // 2] = bytearray(struct.pack("<I", 0x7F800000 if j == 0 else 0x7FC00000))
            elif typ in (1, 30):
                blocks[per_row // 2] = bytearray(struct.pack("<H", bad if typ == 1 else (0x7F80 if j == 0 else 0x7FC0)))
            else:
                blocks[1][0:2] = struct.pack("<H", bad)
            record(f"nonfinite_{tag}_{j}", b"".join(bytes(b) for b in blocks), typ, 1, cols)
            if typ in (3, 7):
                blocks = [bytearray(other_block(typ, rng)) for _ in range(per_row)]
                blocks[2][2:4] = struct.pack("<H", bad)
                record(f"nonfinite_min_{tag}_{j}", b"".join(bytes(b) for b in blocks), typ, 1, cols)
    record("overflow_f32", struct.pack("<I", 0x7F7FFFFF) * 32 + struct.pack("<f", 70000.0) * 32, 0, 2, 32)

    np.savez_compressed(OUT / "other_golden.npz", **arrays)
    (OUT / "other_golden.json").write_text(json.dumps(manifest, indent=1, sort_keys=True) + "\n")
    print(f"wrote {len(manifest)} other-type cases, {sum(a.nbytes for a in arrays.values())} bytes uncompressed")


if __name__ == "__main__":
    main()
    main_other()
