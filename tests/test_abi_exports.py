"""CPU: the C-ABI library loads, exports every function include/tc_qlinear.h declares, and
rejects bad arguments on the host (status codes and messages of the reference's
conventions, native/api/c_api.mm:79-90) without touching a device."""
from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from turbocider_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tc_qlinear.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:[\w]+[\s\*]+)+?(tc_\w+)\s*\(", text, flags=re.M)))


def test_header_declarations_match_binding():
    names = declared_functions()
    assert set(names) == set(_lib.EXPORTS), names


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\sT\s(tc_\w+)", out))
    for name in declared_functions():
        assert name in exported, name
        assert getattr(L, name) is not None


def test_abi_version():
    assert _lib.lib().tc_qlinear_abi_version() == 1


def _decode_status(**kw):
    L = _lib.lib()
    args = dict(type=12, source=0x1000, source_bytes=144, source_rows=1, source_columns=256, row_begin=0, rows=1,
                column_begin=0, columns=256, dtype=2, target=0x100000, target_bytes=512, row_stride=512,
                column_stride=2, idx=None, cancel=None)
    args.update(kw)
    msg = C.c_void_p()
    st = L.tc_gguf_decode_device(args["type"], args["source"], args["source_bytes"], args["source_rows"],
                                 args["source_columns"], args["row_begin"], args["rows"], args["column_begin"],
                                 args["columns"], args["dtype"], args["target"], args["target_bytes"],
                                 args["row_stride"], args["column_stride"], args["idx"], args["cancel"], None, None,
                                 C.byref(msg))
    text = C.cast(msg, C.c_char_p).value.decode() if msg.value else ""
    if msg.value:
        L.tc_qlinear_string_free(msg)
    return st, text


@pytest.mark.parametrize("override,message", [
    (dict(type=9), "gguf_decode: unsupported tensor type"),
    (dict(dtype=99), "gguf_decode: invalid target dtype"),
    (dict(source_columns=255), "invalid source geometry"),
    (dict(rows=2), "row slice out of bounds"),
    (dict(column_begin=250, columns=7), "invalid decode slice"),
    (dict(source_bytes=143), "packed source too short"),
    (dict(column_stride=1), "invalid/overlapping column stride"),
    (dict(row_stride=3), "invalid/overlapping row stride"),
    (dict(target_bytes=511), "decode target too short"),
    (dict(target=0x1000 + 64), "packed source overlaps target"),
    (dict(source=0), "null source/target storage"),
    (dict(source_rows=1 << 62, source_columns=1 << 40, rows=1), "gguf_decode: multiplication overflow"),
])
def test_decode_rejects_bad_geometry_on_host(override, message):
    st, text = _decode_status(**override)
    assert st == 1 and text == message


def test_decode_cancel_and_gather_bounds():
    flag = C.c_int(1)
    assert _decode_status(cancel=C.byref(flag)) == (2, "gguf_decode_cancelled")
    idx = (C.c_uint64 * 2)(0, 1)
    assert _decode_status(idx=idx, rows=2, target_bytes=1024) == (1, "gather row out of bounds")


def test_create_and_forward_reject_bad_arguments():
    L = _lib.lib()
    h = C.c_void_p()
    for desc, message in [
        (_lib.tc_qlinear_desc(9, 16, 256, 0x1000, 1 << 20, None, 0), "unsupported tensor type"),
        (_lib.tc_qlinear_desc(12, 16, 100, 0x1000, 1 << 20, None, 0), "invalid linear geometry"),
        (_lib.tc_qlinear_desc(12, 16, 256, None, 1 << 20, None, 0), "null weight"),
        (_lib.tc_qlinear_desc(12, 16, 256, 0x1000, 100, None, 0), "weight buffer too short"),
        (_lib.tc_qlinear_desc(12, 16, 256, 0x1001, 1 << 20, None, 0), "16-byte aligned"),
        (_lib.tc_qlinear_desc(12, 16, 256, 0x1000, 1 << 20, None, 7), "invalid bias dtype"),
    ]:
        with pytest.raises(_lib.NativeError, match=message):
            _lib.call(L.tc_qlinear_create, C.byref(desc), C.byref(h))
        assert h.value is None
    with pytest.raises(_lib.NativeError, match="null handle"):
        _lib.call(L.tc_qlinear_forward, None, 0x1000, 1, 256, 0x2000, 16, None, 0, None)
    with pytest.raises(_lib.NativeError, match="null handle"):
        _lib.call(L.tc_qlinear_set_path, None, 1)
    L.tc_qlinear_free(None)


def test_quantize_rejects_bad_arguments():
    L = _lib.lib()
    with pytest.raises(_lib.NativeError, match="unsupported quantize type"):
        _lib.call(L.tc_gguf_quantize_device, 13, 0x1000, 1, 256, 0x2000, 176, None)
    with pytest.raises(_lib.NativeError, match="quantize target too short"):
        _lib.call(L.tc_gguf_quantize_device, 12, 0x1000, 2, 256, 0x2000, 200, None)
