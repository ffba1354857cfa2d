"""GGUF container reader (tc_gguf_* C ABI) on the CPU: directory parse, metadata, validation.

The edge cases are those the reference's directory tests cover (tests/native/
test_gguf_execution.py:130-175: every registered type, bounds / alignment / duplicates /
overlap / block alignment, metadata arrays and booleans, split sets); the expected reasons are
tc::gguf::read_directory's error contract (native/core/gguf_directory.hpp:199-304). Files are
assembled by ``GGUFImage`` below from the GGUF v2/v3 layout: header, typed key/value pairs,
tensor descriptors, then the payload section at the aligned data offset. Directory parsing is
host code, so these run without a GPU.
"""
from __future__ import annotations

import struct

import pytest

from turbocider_amd import _lib
from turbocider_amd.gguf import TYPES

GGUF_MAGIC = 0x46554747  # "GGUF" little-endian

# GGUF metadata value types -> struct codes of the fixed-width ones.
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_PACK = {U8: "B", I8: "b", U16: "H", I16: "h", U32: "I", I32: "i", F32: "f", BOOL: "B", U64: "Q", I64: "q",
         F64: "d"}


def lp(text: str) -> bytes:
    """A GGUF string: u64 byte length, then the UTF-8 bytes."""
    raw = text.encode()
    return len(raw).to_bytes(8, "little") + raw


def kv(key: str, vtype: int, value) -> bytes:
    """One key/value pair with a scalar or string value."""
    payload = lp(value) if vtype == STRING else struct.pack("<" + _PACK[vtype], value)
    return lp(key) + vtype.to_bytes(4, "little") + payload


def kv_array(key: str, element_type: int, items: list[bytes]) -> bytes:
    """An array pair whose elements are already encoded (strings via lp, nested arrays, ...)."""
    return lp(key) + ARRAY.to_bytes(4, "little") + element_type.to_bytes(4, "little") + \
        len(items).to_bytes(8, "little") + b"".join(items)


class GGUFImage:
    """Builds a GGUF file image in memory.

    Tensors are placed back to back at `alignment` unless an explicit relative offset is
    given; ``build(data=False)`` leaves the payload section out (the directory alone)."""

    def __init__(self, version: int = 3, magic: int = GGUF_MAGIC, alignment: int = 32):
        self.version, self.magic, self.alignment = version, magic, alignment
        self.pairs: list[bytes] = []
        self.tensors: list[tuple] = []  # (name, type, dims, offset or None, payload or None)

    def meta(self, *pairs: bytes) -> "GGUFImage":
        self.pairs.extend(pairs)
        return self

    def tensor(self, name: str, ggml_type: int, dims, offset: int | None = None, payload: bytes | None = None):
        self.tensors.append((name, ggml_type, list(dims), offset, payload))
        return self

    @staticmethod
    def payload_bytes(ggml_type: int, dims) -> int:
        count = 1
        for d in dims:
            count *= d
        t = TYPES.get(ggml_type)
        return count // t.elements * t.bytes if t else count

    def build(self, data: bool = True) -> bytes:
        descriptors, placed, cursor = [], [], 0
        for name, typ, dims, offset, payload in self.tensors:
            at = cursor if offset is None else offset
            size = self.payload_bytes(typ, dims)
            descriptors.append(lp(name) + len(dims).to_bytes(4, "little") +
                               b"".join(d.to_bytes(8, "little") for d in dims) +
                               typ.to_bytes(4, "little") + at.to_bytes(8, "little"))
            placed.append((at, size, payload))
            cursor = -(-(at + size) // self.alignment) * self.alignment
        head = (self.magic.to_bytes(4, "little") + self.version.to_bytes(4, "little") +
                len(self.tensors).to_bytes(8, "little") + len(self.pairs).to_bytes(8, "little") +
                b"".join(self.pairs) + b"".join(descriptors))
        head += bytes(-len(head) % self.alignment)
        if not data:
            return head
        body = bytearray(max((at + size for at, size, _ in placed), default=0))
        for at, size, payload in placed:
            if payload is not None:
                body[at:at + size] = payload
        return head + bytes(body)


def image(*tensors, pairs=(), **kw) -> GGUFImage:
    img = GGUFImage(**kw).meta(*pairs)
    for t in tensors:
        img.tensor(*t)
    return img


@pytest.fixture()
def gfile(tmp_path):
    from turbocider_amd import gguf_file

    def make(raw: bytes, name="f.gguf"):
        p = tmp_path / name
        p.write_bytes(raw)
        return gguf_file.GGUFFile(p)
    return make


def test_every_registered_type_parses_with_block_geometry(gfile):
    for typ, info in TYPES.items():
        cols = max(info.elements, 32)
        f = gfile(image(("w", typ, [cols, 3])).build())
        t = f.tensor("w")
        assert (t.ggml_type, t.dims, t.elements) == (typ, (cols, 3), 3 * cols)
        assert t.bytes == 3 * cols // info.elements * info.bytes
        assert t.file_offset == f.data_offset and f.data_offset % 32 == 0 and f.version == 3
        assert t.shape == (3, cols)
        f.close()


def test_offsets_alignment_and_metadata_values(gfile):
    pairs = [kv("general.alignment", U32, 64), kv("general.architecture", STRING, "qwen_image"),
             kv("u8", U8, 200), kv("i8", I8, -5), kv("u16", U16, 65535), kv("i16", I16, -300),
             kv("i32", I32, -70000), kv("f32", F32, 1.5), kv("flag", BOOL, 1), kv("u64", U64, 2**40 + 3),
             kv("i64", I64, -(2**40)), kv("f64", F64, -0.25),
             kv_array("tokens", STRING, [lp("a"), lp("bc")]),
             kv_array("nested", ARRAY, [struct.pack("<IQII", U32, 2, 1, 2)])]
    f = gfile(image(("blk.0.attn_q.weight", 12, [512, 4]), ("blk.0.attn_q.bias", 0, [4]),
                    ("blk.0.ffn_down.weight", 14, [256, 2]), pairs=pairs, alignment=64).build())
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
    assert f.metadata("tokens") == {"element_type": STRING, "count": 2}
    assert f.metadata("nested") == {"element_type": ARRAY, "count": 1}
    assert f.projection_prefixes() == ["blk.0.attn_q", "blk.0.ffn_down"]
    with pytest.raises(_lib.NativeError, match="gguf_metadata_missing: nope"):
        f.metadata("nope")
    with pytest.raises(_lib.NativeError, match="gguf_tensor_missing: nope"):
        f.tensor("nope")


def _w8(*extra_pairs, **kw):
    """A one-tensor Q8_0 file with extra metadata pairs."""
    return image(("w", 8, [32]), pairs=extra_pairs, **kw).build()


@pytest.mark.parametrize("raw,reason", [
    (image(("w", 8, [32, 2])).build()[:-1], "tensor payload out of file bounds"),
    (image(("w", 8, [32], 1)).build(), "unaligned tensor offset"),
    (image(("w", 8, [32]), ("w", 8, [32])).build(), "duplicate tensor name"),
    (image(("a", 8, [32], 0), ("b", 8, [32], 0)).build(), "overlapping tensor payloads"),
    (image(("w", 8, [31])).build(), "continuous dimension is not block aligned"),
    (image(("w", 12, [32])).build(), "continuous dimension is not block aligned"),
    (image(("w", 0, [0])).build(), "invalid tensor dimension"),
    (image(("w", 0, [2**32])).build(data=False), "invalid tensor dimension"),
    (_w8(kv("general.alignment", U32, 3)), "invalid alignment"),
    (_w8(kv("general.alignment", U64, 64)), "alignment must be uint32"),
    (_w8(kv("k", U32, 1), kv("k", U32, 2)), "duplicate metadata key"),
    (_w8(kv("bool", BOOL, 2)), "invalid boolean"),
    (_w8(kv_array("ba", BOOL, [b"\x02"])), "invalid boolean"),
    (_w8(lp("big") + struct.pack("<IIQ", ARRAY, U8, 2**21)), "array element limit"),
    (_w8(lp("e") + struct.pack("<IIQ", ARRAY, 13, 1)), "invalid array element type"),
    (_w8(lp("x") + struct.pack("<I", 13)), "invalid metadata scalar type"),
    (_w8(lp("") + struct.pack("<IB", U8, 1)), "invalid metadata key"),
    (image(("w", 0, [1, 1, 1, 1, 1])).build(), "invalid tensor rank"),
    (_w8(magic=0x46554748), "invalid GGUF magic/endian"),
    (_w8(version=1), "unsupported GGUF version"),
    (image().build(), "tensor count limit"),
    (_w8()[:20], "truncated directory"),
    (_w8(lp("s") + struct.pack("<IQ", STRING, 10_000)), "truncated string"),
    (_w8(lp("s") + struct.pack("<IQ", STRING, (1 << 20) + 1)), "string byte limit"),
    (image(("", 8, [32])).build(), "invalid tensor name"),
])
def test_invalid_directories_are_rejected_with_the_reference_reason(gfile, raw, reason):
    with pytest.raises(_lib.NativeError, match="gguf_invalid: " + reason):
        gfile(raw)


def test_nested_array_depth_limit(gfile):
    """Arrays nested five deep: the fifth level exceeds the depth limit of 4."""
    inner = struct.pack("<IQ", U8, 0)
    for _ in range(4):
        inner = struct.pack("<IQ", ARRAY, 1) + inner
    with pytest.raises(_lib.NativeError, match="gguf_invalid: nested array depth limit"):
        gfile(_w8(lp("deep") + ARRAY.to_bytes(4, "little") + inner))
    # Four levels are accepted.
    ok = struct.pack("<IQ", U8, 0)
    for _ in range(3):
        ok = struct.pack("<IQ", ARRAY, 1) + ok
    gfile(_w8(lp("deep") + ARRAY.to_bytes(4, "little") + ok)).close()


def test_skipped_arrays_of_strings_and_booleans(gfile):
    """Array payloads are skipped element by element (strings, booleans, nested arrays of
    scalars), and parsing continues at the right offset."""
    nested = kv_array("n", ARRAY, [struct.pack("<IQ", U16, 3) + struct.pack("<3H", 1, 2, 3),
                                   struct.pack("<IQ", STRING, 2) + lp("x") + lp("yz")])
    f = gfile(_w8(kv_array("flags", BOOL, [b"\x00", b"\x01"]), nested, kv("after", U32, 7)))
    assert f.metadata("flags") == {"element_type": BOOL, "count": 2}
    assert f.metadata("n") == {"element_type": ARRAY, "count": 2}
    assert f.metadata("after") == 7
    f.close()


def test_unsupported_type_id(gfile):
    with pytest.raises(_lib.NativeError, match="gguf_type_unsupported: 99"):
        gfile(image(("w", 99, [32])).build())


def test_first_error_order(gfile):
    """Where a file breaks several rules, the one the reference meets first is reported: the
    duplicate key (checked right after the key) before its malformed value, the tensor-name
    duplicate before a bad rank, and payload bounds (directory order) before overlap."""
    with pytest.raises(_lib.NativeError, match="duplicate metadata key"):
        gfile(_w8(kv("k", U32, 1), lp("k") + struct.pack("<I", 13)))
    with pytest.raises(_lib.NativeError, match="duplicate tensor name"):
        gfile(image(("w", 8, [32]), ("w", 8, [32])).build())
    img = image(("a", 8, [32], 0), ("b", 8, [32], 0), ("c", 8, [32], 1 << 20))
    with pytest.raises(_lib.NativeError, match="tensor payload out of file bounds"):
        gfile(img.build()[:-1])


def split_shard(number, count=2, total=2, arch="qwen3", name=None, count_type=I32):
    pairs = [kv("split.no", U16, number), kv("split.count", U16, count), kv("split.tensors.count", count_type, total),
             kv("general.architecture", STRING, arch)]
    return image((name or f"w{number}", 8, [32]), pairs=pairs).build()


def test_split_sets(gfile):
    from turbocider_amd import gguf_file
    first = gfile(split_shard(0), "a.gguf")
    gguf_file.validate_split([first, gfile(split_shard(1, count_type=U64), "b.gguf")])
    for raw, reason in [(split_shard(0), "duplicate split number"),
                        (split_shard(1, arch="other"), "inconsistent split architecture"),
                        (split_shard(1, total=3), "inconsistent split tensor count"),
                        (split_shard(1, name="w0"), "duplicate split tensor"),
                        (split_shard(1, count=3), "missing split shard or invalid split number"),
                        (split_shard(1, arch=""), "missing split architecture")]:
        with pytest.raises(_lib.NativeError, match=reason):
            gguf_file.validate_split([first, gfile(raw, "c.gguf")])
    with pytest.raises(_lib.NativeError, match="missing split shard"):
        gguf_file.validate_split([first])
    with pytest.raises(_lib.NativeError, match="split tensor count mismatch"):
        gguf_file.validate_split([gfile(split_shard(0, total=3), "d.gguf"), gfile(split_shard(1, total=3), "e.gguf")])
    with pytest.raises(_lib.NativeError, match="negative split tensor count"):
        gguf_file.validate_split([gfile(split_shard(0, total=-2), "f.gguf"), gfile(split_shard(1), "g.gguf")])
    gguf_file.validate_split([gfile(image(("w", 8, [32])).build(), "lone.gguf")])


def test_split_set_aggregate_retained_limit(gfile):
    """The shards' retained directory bytes together must stay within one file's budget
    (32 MiB): three shards that each retain about 11.5 MiB of metadata text are rejected."""
    from turbocider_amd import gguf_file
    text = "x" * ((1 << 20) - 64)
    shards = []
    for i in range(3):
        pairs = [kv(f"blob{j}", STRING, text) for j in range(11)]
        pairs += [kv("split.no", U16, i), kv("split.count", U16, 3), kv("split.tensors.count", I32, 3),
                  kv("general.architecture", STRING, "qwen3")]
        shards.append(gfile(image((f"w{i}", 8, [32]), pairs=pairs).build(), f"s{i}.gguf"))
    with pytest.raises(_lib.NativeError, match="aggregate split metadata limit"):
        gguf_file.validate_split(shards)
    gguf_file.validate_split([gfile(split_shard(0, count=1, total=1), "one.gguf")])


# -- all-or-nothing projection loading (GgufPackedBank::load_candidate,
#    native/runtime/streaming/gguf_packed_bank.cpp:374-515): host logic only; the per-tensor
#    upload is replaced by a recorder, the device path is covered by test_gpu_gguf_file.py.
def _three_projection_file(gfile):
    return gfile(image(("a.weight", 12, [256, 2]), ("b.weight", 12, [256, 2]), ("c.weight", 14, [256, 2])).build())


def _recording(f, fail_at=None):
    calls = []

    def candidate(prefix):
        calls.append(prefix)
        if prefix == fail_at:
            raise _lib.NativeError(f"upload of {prefix} failed")
        return prefix, object()
    f._candidate = candidate
    return calls


def test_load_projections_publishes_all_at_once(gfile, monkeypatch):
    from turbocider_amd import gguf_file, qlinear
    monkeypatch.setattr(gguf_file.torch.cuda, "synchronize", lambda: None)
    f = _three_projection_file(gfile)
    calls = _recording(f)
    events = []
    w = qlinear.Weights()
    assert f.load_projections(w, event=lambda *e: events.append(e)) == ["a", "b", "c"]
    assert calls == ["a", "b", "c"] and w.bound_prefixes() == ["a", "b", "c"]
    assert events == [("load_gguf_direct_tensor", i, 3) for i in range(4)]
    # A second load into the same (non-empty) output is refused before any upload.
    with pytest.raises(_lib.NativeError, match="fresh bank and empty output"):
        f.load_projections(w)
    assert calls == ["a", "b", "c"]


def test_load_projections_failure_binds_nothing(gfile, monkeypatch):
    from turbocider_amd import gguf_file, qlinear
    monkeypatch.setattr(gguf_file.torch.cuda, "synchronize", lambda: None)
    f = _three_projection_file(gfile)
    calls = _recording(f, fail_at="c")
    w = qlinear.Weights()
    with pytest.raises(_lib.NativeError, match="upload of c failed"):
        f.load_projections(w)
    assert calls == ["a", "b", "c"] and w.bound_prefixes() == []
    with pytest.raises(_lib.NativeError, match="duplicate projection prefix"):
        f.load_projections(w, ["a", "a"])


def test_load_projections_cancel_binds_nothing(gfile, monkeypatch):
    import threading
    from turbocider_amd import gguf_file, qlinear
    monkeypatch.setattr(gguf_file.torch.cuda, "synchronize", lambda: None)
    f = _three_projection_file(gfile)
    calls = _recording(f)
    stop = threading.Event()
    w = qlinear.Weights()
    # Cancelled from the progress event of the second tensor: the poll after the event stops it.
    with pytest.raises(gguf_file.LoadCancelled):
        f.load_projections(w, event=lambda name, done, total: stop.set() if done == 1 else None, cancel=stop)
    assert calls == ["a"] and w.bound_prefixes() == []
    # Cancelled at publication (the last event): everything uploaded, nothing bound.
    calls.clear()
    flag = []
    with pytest.raises(gguf_file.LoadCancelled):
        f.load_projections(w, event=lambda name, done, total: flag.append(1) if done == total else None,
                           cancel=lambda: bool(flag))
    assert calls == ["a", "b", "c"] and w.bound_prefixes() == []


def test_load_projections_source_changed(gfile, monkeypatch, tmp_path):
    import os
    from turbocider_amd import gguf_file, qlinear
    monkeypatch.setattr(gguf_file.torch.cuda, "synchronize", lambda: None)
    f = _three_projection_file(gfile)
    calls = _recording(f)
    st = os.stat(f.path)
    w = qlinear.Weights()

    def touch(name, done, total):
        if done == 2:
            os.utime(f.path, ns=(st.st_atime_ns, st.st_mtime_ns + 1_000_000_000))
    with pytest.raises(_lib.NativeError, match="source changed"):
        f.load_projections(w, event=touch)
    # The change lands after the check that precedes tensor c: c is uploaded, publication refused.
    assert w.bound_prefixes() == [] and calls == ["a", "b", "c"]
