"""GGUF container reader (tc_gguf_* C ABI) on the CPU: directory parse, metadata, validation.

The cases restate the reference's own directory tests (tests/native/test_gguf_execution.py:
130-175: every registered type, bounds / alignment / duplicates / overlap / block alignment,
metadata arrays and booleans, split sets) against tc::gguf::read_directory's checks
(native/core/gguf_directory.hpp:199-304), on fixtures written by the small GGUF writer below.
Directory parsing is host code, so these run without a GPU.
"""
from __future__ import annotations

import math
import struct

import pytest

from turbocider_amd import _lib

TYPES = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
         12: (256, 144), 13: (256, 176), 14: (256, 210), 30: (1, 2)}


def gstr(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def meta(key: str, typ: int, value) -> bytes:
    fmt = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "B", 10: "Q", 11: "q", 12: "d"}
    body = gstr(value) if typ == 8 else struct.pack("<" + fmt[typ], value)
    return gstr(key) + struct.pack("<I", typ) + body


def write_gguf(tensors, metas=(), alignment=32, version=3, magic=0x46554747, payload=None, pad_payload=True):
    """tensors: (name, type, dims (GGML order), [relative offset]); payload: optional bytes per
    tensor (default zeros)."""
    head = struct.pack("<IIQQ", magic, version, len(tensors), len(metas)) + b"".join(metas)
    offset, end, placed = 0, 0, []
    for i, t in enumerate(tensors):
        name, typ, dims = t[:3]
        pos = t[3] if len(t) > 3 else offset
        el, bb = TYPES.get(typ, (1, 1))
        size = math.prod(dims) // el * bb
        head += gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", typ, pos)
        placed.append((pos, size))
        offset = (pos + size + alignment - 1) // alignment * alignment
        end = max(end, pos + size)
    head += bytes((-len(head)) % alignment)
    data = bytearray(min(end, 1 << 20) if pad_payload else 0)
    if payload:
        for (pos, size), blob in zip(placed, payload):
            data[pos:pos + size] = blob
    return head + bytes(data)


@pytest.fixture()
def gfile(tmp_path):
    from turbocider_amd import gguf_file
    paths = []

    def make(raw: bytes, name="f.gguf"):
        p = tmp_path / name
        p.write_bytes(raw)
        paths.append(p)
        return gguf_file.GGUFFile(p)
    return make


def test_every_registered_type_parses_with_block_geometry(gfile):
    for typ, (el, bb) in TYPES.items():
        cols = max(el, 32)
        f = gfile(write_gguf([("w", typ, [cols, 3])]))
        t = f.tensor("w")
        assert (t.ggml_type, t.dims, t.elements) == (typ, (cols, 3), 3 * cols)
        assert t.bytes == 3 * cols // el * bb
        assert t.file_offset == f.data_offset and f.data_offset % 32 == 0 and f.version == 3
        assert t.shape == (3, cols)
        f.close()


def test_offsets_alignment_and_metadata_values(gfile):
    metas = [meta("general.alignment", 4, 64), meta("general.architecture", 8, "qwen_image"),
             meta("u8", 0, 200), meta("i8", 1, -5), meta("u16", 2, 65535), meta("i16", 3, -300),
             meta("i32", 5, -70000), meta("f32", 6, 1.5), meta("flag", 7, 1), meta("u64", 10, 2**40 + 3),
             meta("i64", 11, -(2**40)), meta("f64", 12, -0.25),
             gstr("tokens") + struct.pack("<IIQ", 9, 8, 2) + gstr("a") + gstr("bc"),
             gstr("nested") + struct.pack("<IIQ", 9, 9, 1) + struct.pack("<IQ", 4, 2) + struct.pack("<II", 1, 2)]
    f = gfile(write_gguf([("blk.0.attn_q.weight", 12, [512, 4]), ("blk.0.attn_q.bias", 0, [4]),
                          ("blk.0.ffn_down.weight", 14, [256, 2])], metas, alignment=64))
    assert f.alignment == 64 and f.data_offset % 64 == 0
    q = f.tensor("blk.0.attn_q.weight")
    b = f.tensor("blk.0.attn_q.bias")
    d = f.tensor("blk.0.ffn_down.weight")
    assert q.bytes == 4 * 2 * 144 and b.bytes == 16 and d.bytes == 2 * 210
    assert b.file_offset == q.file_offset + 1152 and d.file_offset == b.file_offset + 64
    assert f.metadata("general.architecture") == "qwen_image"
    assert (f.metadata("u8"), f.metadata("i8"), f.metadata("u16"), f.metadata("i16")) == (200, -5, 65535, -300)
    assert (f.metadata("i32"), f.metadata("f32"), f.metadata("flag")) == (-70000, 1.5, True)
    assert (f.metadata("u64"), f.metadata("i64"), f.metadata("f64")) == (2**40 + 3, -(2**40), -0.25)
    assert f.metadata("tokens") == {"element_type": 8, "count": 2}
    assert f.metadata("nested") == {"element_type": 9, "count": 1}
    assert f.projection_prefixes() == ["blk.0.attn_q", "blk.0.ffn_down"]
    with pytest.raises(_lib.NativeError, match="gguf_metadata_missing: nope"):
        f.metadata("nope")
    with pytest.raises(_lib.NativeError, match="gguf_tensor_missing: nope"):
        f.tensor("nope")


@pytest.mark.parametrize("raw,reason", [
    (write_gguf([("w", 8, [32, 2])])[:-1], "tensor payload out of file bounds"),
    (write_gguf([("w", 8, [32], 1)]), "unaligned tensor offset"),
    (write_gguf([("w", 8, [32]), ("w", 8, [32])]), "duplicate tensor name"),
    (write_gguf([("a", 8, [32], 0), ("b", 8, [32], 0)]), "overlapping tensor payloads"),
    (write_gguf([("w", 8, [31])]), "continuous dimension is not block aligned"),
    (write_gguf([("w", 12, [32])]), "continuous dimension is not block aligned"),
    (write_gguf([("w", 0, [0])]), "invalid tensor dimension"),
    (write_gguf([("w", 0, [2**32])])[:256], "invalid tensor dimension"),
    (write_gguf([("w", 8, [32])], [meta("general.alignment", 4, 3)]), "invalid alignment"),
    (write_gguf([("w", 8, [32])], [meta("general.alignment", 10, 64)]), "alignment must be uint32"),
    (write_gguf([("w", 8, [32])], [meta("k", 4, 1), meta("k", 4, 2)]), "duplicate metadata key"),
    (write_gguf([("w", 8, [32])], [meta("bool", 7, 2)]), "invalid boolean"),
    (write_gguf([("w", 8, [32])], [gstr("ba") + struct.pack("<IIQB", 9, 7, 1, 2)]), "invalid boolean"),
    (write_gguf([("w", 8, [32])], [gstr("big") + struct.pack("<IIQ", 9, 0, 2**21)]), "array element limit"),
    (write_gguf([("w", 8, [32])], [gstr("e") + struct.pack("<IIQ", 9, 13, 1)]), "invalid array element type"),
    (write_gguf([("w", 8, [32])], [gstr("x") + struct.pack("<I", 13)]), "invalid metadata scalar type"),
    (write_gguf([("w", 8, [32])], [gstr("") + struct.pack("<IB", 0, 1)]), "invalid metadata key"),
    (write_gguf([("w", 0, [1, 1, 1, 1, 1])]), "invalid tensor rank"),
    (write_gguf([("w", 8, [32])], magic=0x46554748), "invalid GGUF magic/endian"),
    (write_gguf([("w", 8, [32])], version=1), "unsupported GGUF version"),
    (write_gguf([]), "tensor count limit"),
    (write_gguf([("w", 8, [32])])[:20], "truncated directory"),
])
def test_invalid_directories_are_rejected_with_the_reference_reason(gfile, raw, reason):
    with pytest.raises(_lib.NativeError, match="gguf_invalid: " + reason):
        gfile(raw)


def test_nested_array_depth_limit(gfile):
    deep = gstr("deep") + struct.pack("<IIQ", 9, 9, 1)
    for _ in range(4):
        deep += struct.pack("<IQ", 9, 1)
    deep += struct.pack("<IQ", 0, 0)
    with pytest.raises(_lib.NativeError, match="gguf_invalid: nested array depth limit"):
        gfile(write_gguf([("w", 8, [32])], [deep]))


def test_unsupported_type_id(gfile):
    with pytest.raises(_lib.NativeError, match="gguf_type_unsupported: 99"):
        gfile(write_gguf([("w", 99, [32])]))


def test_split_sets(gfile):
    from turbocider_amd import gguf_file

    def shard(number, count=2, total=2, arch="qwen3", name=None):
        m = [meta("split.no", 2, number), meta("split.count", 2, count), meta("split.tensors.count", 5, total),
             meta("general.architecture", 8, arch)]
        return write_gguf([(name or f"w{number}", 8, [32])], m)

    first = gfile(shard(0), "a.gguf")
    gguf_file.validate_split([first, gfile(shard(1), "b.gguf")])
    for raw, reason in [(shard(0), "duplicate split number"), (shard(1, arch="other"), "inconsistent split architecture"),
                        (shard(1, total=3), "inconsistent split tensor count"), (shard(1, name="w0"), "duplicate split tensor")]:
        with pytest.raises(_lib.NativeError, match=reason):
            gguf_file.validate_split([first, gfile(raw, "c.gguf")])
    with pytest.raises(_lib.NativeError, match="missing split shard"):
        gguf_file.validate_split([first])
    gguf_file.validate_split([gfile(write_gguf([("w", 8, [32])]), "lone.gguf")])
