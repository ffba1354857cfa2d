"""GGUF tensor formats and the device decoder.

Mirrors the reference's decode interface (native/core/gguf_decode.hpp:10-65): a
``PackedMatrix`` (raw GGUF bytes + GGML type + logical rows/columns), a ``DecodeSlice``, a
``DecodeTarget`` (bytes + dtype + byte strides), ``decode_into`` / ``decode_gather`` and a
``DecodeError`` on any rejected geometry or non-finite scale. Here every tensor lives in GPU
memory (torch tensors on a HIP device) and the work runs in ``libtc_qlinear.so``.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from enum import IntEnum

import torch

from . import _lib


@dataclass(frozen=True)
class TypeInfo:
    """GGML type registry entry (native/core/gguf_directory.hpp:19-26)."""
    id: int
    elements: int
    bytes: int
    name: str


F32 = TypeInfo(0, 1, 4, "F32")
F16 = TypeInfo(1, 1, 2, "F16")
Q4_0 = TypeInfo(2, 32, 18, "Q4_0")
Q4_1 = TypeInfo(3, 32, 20, "Q4_1")
Q5_0 = TypeInfo(6, 32, 22, "Q5_0")
Q5_1 = TypeInfo(7, 32, 24, "Q5_1")
Q8_0 = TypeInfo(8, 32, 34, "Q8_0")
Q4_K = TypeInfo(12, 256, 144, "Q4_K")
Q5_K = TypeInfo(13, 256, 176, "Q5_K")
Q6_K = TypeInfo(14, 256, 210, "Q6_K")
BF16 = TypeInfo(30, 1, 2, "BF16")
# Every type the decoder takes; the quantized projection reads Q4_K, Q5_K and Q6_K directly.
TYPES = {t.id: t for t in (F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, BF16)}


def type_info(type_id: int) -> TypeInfo:
    if type_id not in TYPES:
        raise ValueError(f"gguf_type_unsupported: {type_id}")
    return TYPES[type_id]


def row_bytes(type_id: int, columns: int) -> int:
    t = type_info(type_id)
    if columns % t.elements:
        raise ValueError("invalid source geometry")
    return columns // t.elements * t.bytes


class DecodeDType(IntEnum):
    """Target element type (gguf_decode.hpp:18)."""
    f32 = 0
    f16 = 1
    bf16 = 2


def dtype_bytes(dtype: DecodeDType) -> int:
    return 4 if dtype == DecodeDType.f32 else 2


class DecodeError(RuntimeError):
    """Rejected decode (gguf_decode.hpp:10-16); the target must be discarded."""


class DecodeCancelled(DecodeError):
    pass


@dataclass
class PackedMatrix:
    bytes: torch.Tensor  # uint8 tensor holding the raw blocks (device; host for decode_cpu_*)
    type: int
    rows: int
    columns: int


@dataclass
class DecodeSlice:
    row_begin: int = 0
    rows: int = 0
    column_begin: int = 0
    columns: int = 0


@dataclass
class DecodeTarget:
    bytes: torch.Tensor  # tensor (any dtype) viewed as raw bytes (device; host for decode_cpu_*)
    dtype: DecodeDType = DecodeDType.bf16
    row_stride: int = 0      # bytes
    column_stride: int = 0   # bytes


@dataclass
class DecodeReceipt:
    source_bytes_processed: int = 0
    elements_written: int = 0
    bytes_written: int = 0
    scratch_bytes: int = 0
    simd_blocks: int = 0


def _stream_handle(stream) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _decode(source: PackedMatrix, row_begin: int, rows: int, column_begin: int, columns: int,
            target: DecodeTarget, gather, cancel, stream) -> DecodeReceipt:
    L = _lib.lib()
    receipt = _lib.tc_decode_receipt()
    idx = (C.c_uint64 * len(gather))(*gather) if gather is not None else None
    flag = C.c_int(1) if cancel else None
    try:
        _lib.call(L.tc_gguf_decode_device, source.type, source.bytes.data_ptr(), source.bytes.numel()
                  * source.bytes.element_size(), source.rows, source.columns, row_begin, rows, column_begin, columns,
                  int(target.dtype), target.bytes.data_ptr(), target.bytes.numel() * target.bytes.element_size(),
                  target.row_stride, target.column_stride, idx, C.byref(flag) if flag is not None else None,
                  _stream_handle(stream), C.byref(receipt))
    except _lib.NativeCancelled as e:
        raise DecodeCancelled(str(e)) from None
    except _lib.NativeError as e:
        raise DecodeError(str(e)) from None
    return DecodeReceipt(receipt.source_bytes_processed, receipt.elements_written, receipt.bytes_written,
                         receipt.scratch_bytes, receipt.simd_blocks)


def decode_into(source: PackedMatrix, slice: DecodeSlice, target: DecodeTarget, cancel: bool = False,
                stream=None) -> DecodeReceipt:
    """Device equivalent of tc::gguf::decode_cpu_into (gguf_decode.hpp:56-58). Synchronous."""
    return _decode(source, slice.row_begin, slice.rows, slice.column_begin, slice.columns, target, None, cancel,
                   stream)


def decode_gather(source: PackedMatrix, row_indices, column_begin: int, columns: int, target: DecodeTarget,
                  cancel: bool = False, stream=None) -> DecodeReceipt:
    """Device equivalent of tc::gguf::decode_cpu_gather (gguf_decode.hpp:62-65). Synchronous."""
    rows = [int(r) for r in row_indices]
    return _decode(source, 0, len(rows), column_begin, columns, target, rows, cancel, stream)


def _host_buffer(obj):
    """(address, bytes) of a host buffer: a CPU torch tensor or a numpy array."""
    if isinstance(obj, torch.Tensor):
        if obj.is_cuda:
            raise DecodeError("the host decode takes host (CPU) buffers")
        return obj.data_ptr(), obj.numel() * obj.element_size()
    return obj.ctypes.data, obj.nbytes


def _decode_host(source: PackedMatrix, row_begin: int, rows: int, column_begin: int, columns: int,
                 target: DecodeTarget, gather, cancel) -> DecodeReceipt:
    receipt = _lib.tc_decode_receipt()
    idx = (C.c_uint64 * len(gather))(*gather) if gather is not None else None
    flag = C.c_int(1) if cancel else None
    src, src_bytes = _host_buffer(source.bytes)
    dst, dst_bytes = _host_buffer(target.bytes)
    try:
        _lib.call(_lib.lib().tc_gguf_decode_host, source.type, src, src_bytes, source.rows, source.columns,
                  row_begin, rows, column_begin, columns, int(target.dtype), dst, dst_bytes, target.row_stride,
                  target.column_stride, idx, C.byref(flag) if flag is not None else None, C.byref(receipt))
    except _lib.NativeCancelled as e:
        raise DecodeCancelled(str(e)) from None
    except _lib.NativeError as e:
        raise DecodeError(str(e)) from None
    return DecodeReceipt(receipt.source_bytes_processed, receipt.elements_written, receipt.bytes_written,
                         receipt.scratch_bytes, receipt.simd_blocks)


def decode_cpu_into(source: PackedMatrix, slice: DecodeSlice, target: DecodeTarget,
                    cancel: bool = False) -> DecodeReceipt:
    """tc::gguf::decode_cpu_into (gguf_decode.hpp:56-58) on host buffers (CPU torch tensors or
    numpy arrays), through tc_gguf_decode_host. Synchronous."""
    return _decode_host(source, slice.row_begin, slice.rows, slice.column_begin, slice.columns, target, None, cancel)


def decode_cpu_gather(source: PackedMatrix, row_indices, column_begin: int, columns: int, target: DecodeTarget,
                      cancel: bool = False) -> DecodeReceipt:
    """tc::gguf::decode_cpu_gather (gguf_decode.hpp:62-65) on host buffers. Synchronous."""
    rows = [int(r) for r in row_indices]
    return _decode_host(source, 0, len(rows), column_begin, columns, target, rows, cancel)


_TORCH_DTYPE = {DecodeDType.f32: torch.float32, DecodeDType.f16: torch.float16, DecodeDType.bf16: torch.bfloat16}


def dequantize(blocks: torch.Tensor, type_id: int, rows: int, columns: int,
               dtype: DecodeDType = DecodeDType.bf16, stream=None) -> torch.Tensor:
    """Whole-matrix decode into a new dense [rows, columns] tensor."""
    out = torch.empty((rows, columns), dtype=_TORCH_DTYPE[DecodeDType(dtype)], device=blocks.device)
    item = dtype_bytes(DecodeDType(dtype))
    decode_into(PackedMatrix(blocks, type_id, rows, columns), DecodeSlice(0, rows, 0, columns),
                DecodeTarget(out, DecodeDType(dtype), columns * item, item), stream=stream)
    return out


def quantize(weights: torch.Tensor, type_id: int, stream=None) -> torch.Tensor:
    """fp32 [rows, columns] device tensor -> raw Q4_K/Q6_K blocks (uint8 device tensor).

    The reference has no quantizer; this one derives per-sub-block affine ranges, stores
    6-bit (Q4_K) or int8 (Q6_K) sub-scales under an fp16 super-block scale, and re-derives
    the codes from the stored scales.
    """
    if weights.dtype != torch.float32 or weights.dim() != 2 or not weights.is_contiguous():
        raise ValueError("quantize expects a contiguous fp32 [rows, columns] tensor")
    rows, columns = weights.shape
    out = torch.empty(rows * row_bytes(type_id, columns), dtype=torch.uint8, device=weights.device)
    _lib.call(_lib.lib().tc_gguf_quantize_device, type_id, weights.data_ptr(), rows, columns, out.data_ptr(),
              out.numel(), _stream_handle(stream))
    return out
