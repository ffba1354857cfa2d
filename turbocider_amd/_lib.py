"""ctypes binding of ``libtc_qlinear.so`` (the C ABI in ``include/tc_qlinear.h``).

The reference reaches native code from Python only through ctypes
(tests/native/test_contract.py:13-41, tests/native/test_gguf_execution.py:77-85); this module
does the same. There is no fallback: if the HIP library is missing, importing the operator
modules raises and names the build command.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("TC_QLINEAR_LIB", Path(__file__).resolve().parent / "libtc_qlinear.so"))

STATUS_OK, STATUS_ERROR, STATUS_CANCELLED = 0, 1, 2

# Symbols declared in include/tc_qlinear.h (checked by tests/test_abi_exports.py).
EXPORTS = (
    "tc_qlinear_abi_version", "tc_qlinear_string_free", "tc_gguf_decode_device", "tc_gguf_decode_host", "tc_gguf_quantize_device",
    "tc_qlinear_create", "tc_qlinear_forward", "tc_qlinear_forward_noalloc", "tc_qlinear_forward_act",
    "tc_qlinear_forward_many", "tc_qlinear_forward_group", "tc_qlinear_set_path", "tc_qlinear_plan",
    "tc_qlinear_free",
    "tc_gguf_open", "tc_gguf_close", "tc_gguf_describe", "tc_gguf_tensor", "tc_gguf_find_tensor", "tc_gguf_meta",
    "tc_gguf_validate_split", "tc_gguf_read_tensor",
    "tc_pager_create", "tc_pager_group_layout", "tc_pager_fill", "tc_pager_acquire", "tc_pager_release",
    "tc_pager_get_metrics", "tc_pager_free",
)


class tc_decode_receipt(C.Structure):
    _fields_ = [("source_bytes_processed", C.c_uint64), ("elements_written", C.c_uint64),
                ("bytes_written", C.c_uint64), ("scratch_bytes", C.c_uint64), ("simd_blocks", C.c_uint64)]


class tc_qlinear_desc(C.Structure):
    _fields_ = [("ggml_type", C.c_uint32), ("n", C.c_uint64), ("k", C.c_uint64), ("weight", C.c_void_p),
                ("weight_bytes", C.c_uint64), ("bias", C.c_void_p), ("bias_dtype", C.c_uint32)]


class tc_lora_adapter(C.Structure):
    _fields_ = [("a", C.c_void_p), ("b", C.c_void_p), ("rank", C.c_uint32), ("scale", C.c_float),
                ("row_begin", C.c_uint64), ("row_count", C.c_uint64), ("output_begin", C.c_uint64),
                ("output_end", C.c_uint64)]


class tc_qlinear_plan_info(C.Structure):
    _fields_ = [("kernel", C.c_uint32), ("tail_rows", C.c_uint32), ("workspace_bytes", C.c_uint64)]


class tc_gguf_summary(C.Structure):
    _fields_ = [("version", C.c_uint32), ("alignment", C.c_uint32), ("tensor_count", C.c_uint64),
                ("metadata_count", C.c_uint64), ("file_bytes", C.c_uint64), ("data_offset", C.c_uint64)]


class tc_gguf_tensor_info(C.Structure):
    _fields_ = [("name", C.c_char_p), ("ggml_type", C.c_uint32), ("rank", C.c_uint32), ("dims", C.c_uint64 * 4),
                ("elements", C.c_uint64), ("bytes", C.c_uint64), ("file_offset", C.c_uint64),
                ("relative_offset", C.c_uint64)]


class tc_gguf_meta_value(C.Structure):
    _fields_ = [("type", C.c_uint32), ("element_type", C.c_uint32), ("count", C.c_uint64),
                ("unsigned_value", C.c_uint64), ("signed_value", C.c_int64), ("float_value", C.c_double),
                ("text", C.c_void_p), ("text_bytes", C.c_uint64)]


class tc_pager_ticket(C.Structure):
    _fields_ = [("group", C.c_uint32), ("slot", C.c_uint32), ("generation", C.c_uint64)]


class tc_pager_metrics(C.Structure):
    _fields_ = [("fills", C.c_uint64), ("bytes_read", C.c_uint64), ("read_seconds", C.c_double),
                ("wait_seconds", C.c_double)]


class NativeError(RuntimeError):
    """Status 1 from the C ABI; the message is the library's error string."""


class NativeCancelled(NativeError):
    """Status 2 from the C ABI (cancellation, c_api.mm:85-90)."""


_lib: C.CDLL | None = None


def lib() -> C.CDLL:
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is missing: build it with `python -m turbocider_amd.build` "
                          "(there is no CPU fallback for the quantized-linear path)")
    L = C.CDLL(str(LIB_PATH))
    err = C.POINTER(C.c_char_p)
    L.tc_qlinear_abi_version.restype = C.c_uint32
    L.tc_qlinear_string_free.argtypes = [C.c_void_p]
    L.tc_gguf_decode_device.argtypes = ([C.c_uint32, C.c_void_p] + [C.c_uint64] * 7 + [C.c_uint32, C.c_void_p]
                                        + [C.c_uint64] * 3 + [C.POINTER(C.c_uint64), C.POINTER(C.c_int),
                                                              C.c_void_p, C.POINTER(tc_decode_receipt), C.c_void_p])
    L.tc_gguf_decode_host.argtypes = ([C.c_uint32, C.c_void_p] + [C.c_uint64] * 7 + [C.c_uint32, C.c_void_p]
                                      + [C.c_uint64] * 3 + [C.POINTER(C.c_uint64), C.POINTER(C.c_int),
                                                            C.POINTER(tc_decode_receipt), C.c_void_p])
    L.tc_gguf_quantize_device.argtypes = [C.c_uint32, C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p, C.c_uint64,
                                          C.c_void_p, C.c_void_p]
    L.tc_qlinear_create.argtypes = [C.POINTER(tc_qlinear_desc), C.POINTER(C.c_void_p), C.c_void_p]
    L.tc_qlinear_forward.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p, C.c_uint64,
                                     C.POINTER(tc_lora_adapter), C.c_uint32, C.c_void_p, C.c_void_p]
    L.tc_qlinear_forward_noalloc.argtypes = L.tc_qlinear_forward.argtypes
    L.tc_qlinear_forward_act.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p,
                                         C.c_uint64, C.POINTER(tc_lora_adapter), C.c_uint32, C.c_void_p, C.c_void_p]
    L.tc_qlinear_forward_many.argtypes = [C.POINTER(C.c_void_p), C.c_uint32, C.c_void_p, C.c_uint64, C.c_uint64,
                                          C.POINTER(C.c_void_p), C.POINTER(C.c_uint64), C.c_void_p, C.c_void_p]
    L.tc_qlinear_forward_group.argtypes = [C.POINTER(C.c_void_p), C.c_uint32, C.c_uint32, C.POINTER(C.c_void_p),
                                           C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.POINTER(C.c_void_p),
                                           C.POINTER(C.c_uint64), C.c_void_p, C.POINTER(C.c_uint32), C.c_void_p]
    L.tc_qlinear_set_path.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p]
    L.tc_qlinear_plan.argtypes = [C.c_uint32] + [C.c_uint64] * 4 + [C.c_uint32, C.POINTER(tc_qlinear_plan_info),
                                                                   C.c_void_p]
    L.tc_qlinear_free.argtypes = [C.c_void_p]
    L.tc_gguf_open.argtypes = [C.c_char_p, C.POINTER(C.c_void_p), C.c_void_p]
    L.tc_gguf_close.argtypes = [C.c_void_p]
    L.tc_gguf_describe.argtypes = [C.c_void_p, C.POINTER(tc_gguf_summary)]
    L.tc_gguf_tensor.argtypes = [C.c_void_p, C.c_uint64, C.POINTER(tc_gguf_tensor_info), C.c_void_p]
    L.tc_gguf_find_tensor.argtypes = [C.c_void_p, C.c_char_p, C.POINTER(C.c_uint64), C.c_void_p]
    L.tc_gguf_meta.argtypes = [C.c_void_p, C.c_char_p, C.POINTER(tc_gguf_meta_value), C.c_void_p]
    L.tc_gguf_validate_split.argtypes = [C.POINTER(C.c_void_p), C.c_uint32, C.c_void_p]
    L.tc_gguf_read_tensor.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]
    L.tc_pager_create.argtypes = [C.c_void_p, C.c_uint32, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.c_uint32,
                                  C.POINTER(C.c_void_p), C.c_uint64, C.POINTER(C.c_void_p), C.c_void_p]
    L.tc_pager_group_layout.argtypes = [C.c_void_p, C.c_uint32, C.POINTER(C.c_uint64), C.c_uint32,
                                        C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.c_void_p]
    L.tc_pager_fill.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.POINTER(C.c_int), C.POINTER(tc_pager_ticket),
                                C.c_void_p]
    L.tc_pager_acquire.argtypes = [C.c_void_p, C.POINTER(tc_pager_ticket), C.c_void_p, C.c_void_p]
    L.tc_pager_release.argtypes = [C.c_void_p, C.POINTER(tc_pager_ticket), C.c_void_p, C.c_void_p]
    L.tc_pager_get_metrics.argtypes = [C.c_void_p, C.POINTER(tc_pager_metrics)]
    L.tc_pager_free.argtypes = [C.c_void_p]
    L.tc_pager_free.restype = None
    for name in EXPORTS:
        getattr(L, name).restype = getattr(L, name).restype or C.c_int
    L.tc_qlinear_abi_version.restype = C.c_uint32
    L.tc_qlinear_free.restype = None
    L.tc_gguf_close.restype = None
    L.tc_qlinear_string_free.restype = None
    _lib = L
    return L


def call(fn, *args) -> None:
    """Invoke an ABI function whose last argument is `char **error`; raise on failure."""
    msg = C.c_void_p()
    status = fn(*args, C.byref(msg))
    if status != STATUS_OK:
        text = C.cast(msg, C.c_char_p).value.decode() if msg.value else "unknown error"
        if msg.value:
            lib().tc_qlinear_string_free(msg)
        raise (NativeCancelled if status == STATUS_CANCELLED else NativeError)(text)
