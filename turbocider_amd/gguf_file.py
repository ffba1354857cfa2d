"""GGUF container reader: tensor directory, metadata, raw-block upload, projection binding.

Python face of the ``tc_gguf_*`` C ABI (``include/tc_qlinear.h``), the MI355X counterpart of
the reference's directory reader ``tc::gguf::read_directory`` / ``validate_split_set``
(native/core/gguf_directory.hpp:199-304) and of its packed-bank binding step, which maps a
``<prefix>.weight`` K-quant tensor (and optional ``<prefix>.bias``) to a projection
(native/core/gguf_weights.hpp:66-119, with the ``model.diffusion_model.`` prefix stripped as
in :115-119). The K-quant payload goes to HBM as the raw GGUF blocks (no host decode); the
device kernels consume them directly.

    with GGUFFile("model-Q4_K_M.gguf") as f:
        W = qlinear.Weights()
        for prefix in f.projection_prefixes():
            f.bind_projection(W, prefix)
        y = W.project(x, "transformer_blocks.0.attn.to_q")
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from typing import Iterable

import torch

from . import _lib, gguf

DIFFUSION_PREFIX = "model.diffusion_model."

# GGUF metadata value types.
META_TYPES = {0: "u8", 1: "i8", 2: "u16", 3: "i16", 4: "u32", 5: "i32", 6: "f32", 7: "bool", 8: "string",
              9: "array", 10: "u64", 11: "i64", 12: "f64"}

# Raw element types of non-quantized tensors -> torch dtype (for biases and norms).
_PLAIN = {0: torch.float32, 1: torch.float16, 30: torch.bfloat16}


@dataclass(frozen=True)
class TensorInfo:
    name: str
    ggml_type: int
    dims: tuple  # GGML order: dims[0] is contiguous
    elements: int
    bytes: int
    file_offset: int

    @property
    def shape(self) -> tuple:
        """Logical (row-major) shape, the reverse of the GGML dims (gguf_directory.hpp:67-69)."""
        return tuple(reversed(self.dims))


def canonical_name(name: str) -> str:
    """Tensor name with the diffusion-model prefix removed (gguf_weights.hpp:115-119)."""
    return name[len(DIFFUSION_PREFIX):] if name.startswith(DIFFUSION_PREFIX) else name


class GGUFFile:
    """An open, validated GGUF file (the directory is parsed once; payloads are read on demand)."""

    def __init__(self, path: str):
        L = _lib.lib()
        h = C.c_void_p()
        _lib.call(L.tc_gguf_open, str(path).encode(), C.byref(h))
        self._h = h
        self.path = str(path)
        self._identity = _identity(self.path)
        s = _lib.tc_gguf_summary()
        if L.tc_gguf_describe(h, C.byref(s)) != 0:
            raise _lib.NativeError("tc_gguf_describe failed")
        self.version, self.alignment = s.version, s.alignment
        self.file_bytes, self.data_offset = s.file_bytes, s.data_offset
        self.metadata_count = s.metadata_count
        self.tensors: list[TensorInfo] = []
        for i in range(s.tensor_count):
            t = _lib.tc_gguf_tensor_info()
            _lib.call(L.tc_gguf_tensor, h, i, C.byref(t))
            self.tensors.append(TensorInfo(t.name.decode(), t.ggml_type, tuple(t.dims[:t.rank]), t.elements,
                                           t.bytes, t.file_offset))
        self._index = {t.name: i for i, t in enumerate(self.tensors)}

    # -- lifetime
    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            _lib.lib().tc_gguf_close(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- directory
    def tensor(self, name: str) -> TensorInfo:
        if name not in self._index:
            raise _lib.NativeError(f"gguf_tensor_missing: {name}")
        return self.tensors[self._index[name]]

    def metadata(self, key: str):
        """Scalar metadata as a Python value; arrays as {"element_type", "count"}."""
        v = _lib.tc_gguf_meta_value()
        _lib.call(_lib.lib().tc_gguf_meta, self._h, key.encode(), C.byref(v))
        if v.type == 8:
            return C.string_at(v.text, v.text_bytes).decode("utf-8", errors="replace")
        if v.type == 9:
            return {"element_type": v.element_type, "count": v.count}
        if v.type in (6, 12):
            return v.float_value
        if v.type == 7:
            return bool(v.unsigned_value)
        if v.type in (1, 3, 5, 11):
            return v.signed_value
        return v.unsigned_value

    def projection_prefixes(self) -> list[str]:
        """Canonical prefixes of the 2-D ``<prefix>.weight`` tensors a projection can bind (every
        registered type: K-quants on the fused kernels, the rest decoded to bf16)."""
        out = []
        for t in self.tensors:
            if t.name.endswith(".weight") and t.ggml_type in gguf.TYPES and len(t.dims) == 2:
                out.append(canonical_name(t.name)[: -len(".weight")])
        return out

    # -- payloads
    def read_tensor(self, name: str, stream=None) -> torch.Tensor:
        """Raw payload bytes of `name` in device memory (uint8, as stored in the file)."""
        t = self.tensor(name)
        dst = torch.empty(t.bytes, dtype=torch.uint8, device="cuda")
        s = stream.cuda_stream if stream is not None else torch.cuda.current_stream().cuda_stream
        _lib.call(_lib.lib().tc_gguf_read_tensor, self._h, self._index[name], C.c_void_p(dst.data_ptr()), t.bytes,
                  C.c_void_p(s))
        return dst

    def read_plain(self, name: str) -> torch.Tensor:
        """An F32 / F16 / BF16 tensor as a device tensor of its logical shape."""
        t = self.tensor(name)
        if t.ggml_type not in _PLAIN:
            raise _lib.NativeError(f"{name}: not a plain F32/F16/BF16 tensor (type {t.ggml_type})")
        return self.read_tensor(name).view(_PLAIN[t.ggml_type]).view(t.shape)

    def gather_rows(self, name: str, row_ids, dtype=None, blocks: torch.Tensor | None = None) -> torch.Tensor:
        """Rows `row_ids` (e.g. a prompt's token ids, in order, repeats allowed) of a 2-D tensor
        of any registered type, decoded on the device into a new [len(row_ids), columns] tensor
        (bf16 unless `dtype` says otherwise): the embedding lookup of a text encoder, which
        decodes only the consumed rows (the reference gathers packed rows before its GPU decode,
        native/models/qwen21/gguf_weights.hpp:110-113; decode_cpu_gather, gguf_decode.hpp:62-65).
        `blocks`: the tensor's payload already in device memory (read once, reused per prompt)."""
        t = self.tensor(name)
        if len(t.dims) != 2:
            raise _lib.NativeError(f"{name}: a row gather needs a 2-D tensor (rank {len(t.dims)})")
        columns, rows = t.dims
        dt = gguf.DecodeDType.bf16 if dtype is None else gguf.DecodeDType(dtype)
        src = self.read_tensor(name) if blocks is None else blocks
        ids = [int(r) for r in row_ids]
        out = torch.empty((len(ids), columns), dtype=gguf._TORCH_DTYPE[dt], device=src.device)
        item = gguf.dtype_bytes(dt)
        gguf.decode_gather(gguf.PackedMatrix(src, t.ggml_type, rows, columns), ids, 0, columns,
                           gguf.DecodeTarget(out, dt, columns * item, item))
        return out

    def _find(self, prefix: str, suffix: str) -> str | None:
        for cand in (prefix + suffix, DIFFUSION_PREFIX + prefix + suffix):
            if cand in self._index:
                return cand
        return None

    def bind_projection(self, weights, prefix: str):
        """Upload ``<prefix>.weight`` (shape [N, K], any registered type) and the optional
        ``<prefix>.bias`` and bind them under `prefix` in a ``qlinear.Weights``."""
        wname = self._find(prefix, ".weight")
        if wname is None:
            raise _lib.NativeError(f"gguf_tensor_missing: {prefix}.weight")
        t = self.tensor(wname)
        if t.ggml_type not in gguf.TYPES or len(t.dims) != 2:
            raise _lib.NativeError(f"{wname}: the device projection takes 2-D weights of a registered type "
                                   f"(type {t.ggml_type}, rank {len(t.dims)})")
        k, n = t.dims
        blocks = self.read_tensor(wname)
        bname = self._find(prefix, ".bias")
        bias = self.read_plain(bname).reshape(-1) if bname else None
        if bias is not None and bias.numel() != n:
            raise _lib.NativeError(f"{bname}: {bias.numel()} values for {n} outputs")
        return weights.bind(prefix, blocks, t.ggml_type, n, k, bias)

    def _candidate(self, prefix: str):
        """Upload and validate one projection without binding it: (prefix, QuantizedLinear)."""
        from .qlinear import Weights
        scratch = Weights()
        lin = self.bind_projection(scratch, prefix)
        return prefix, lin

    def load_projections(self, weights, prefixes=None, cancel=None, event=None) -> list[str]:
        """All-or-nothing binding of projections (GgufPackedBank::load_candidate,
        gguf_packed_bank.cpp:374-515): every ``<prefix>.weight`` (default: all of
        projection_prefixes()) is uploaded and validated into a candidate set first; `weights`
        receives the whole set in one step only after every tensor succeeded, the request was
        not cancelled and the file is unchanged since it was opened. On any failure or
        cancellation nothing is bound and the uploaded candidates are released.

        `weights` must hold no projection yet (the reference requires an empty output).
        `cancel`: an object with ``is_set()`` (threading.Event) or a callable, polled before
        each tensor and before publication; raises LoadCancelled. `event(name, done, total)`
        is called before each tensor and once at publication, as the reference's progress
        event ("load_gguf_direct_tensor")."""
        if weights.bound_prefixes():
            raise _lib.NativeError("gguf_packed_bank: load requires fresh bank and empty output")
        names = self.projection_prefixes() if prefixes is None else list(prefixes)
        if len(set(names)) != len(names):
            raise _lib.NativeError("gguf_packed_bank: duplicate projection prefix")
        candidates = []
        for i, prefix in enumerate(names):
            _check_cancel(cancel)
            self._check_unchanged()
            if event is not None:
                event("load_gguf_direct_tensor", i, len(names))
            _check_cancel(cancel)
            candidates.append(self._candidate(prefix))
        _check_cancel(cancel)
        self._check_unchanged()
        torch.cuda.synchronize()
        if event is not None:
            event("load_gguf_direct_tensor", len(names), len(names))
        _check_cancel(cancel)
        self._check_unchanged()
        weights.publish(dict(candidates))
        return names

    def _check_unchanged(self) -> None:
        """The file still has the identity (device, inode, size, mtime) it had when opened."""
        if _identity(self.path) != self._identity:
            raise _lib.NativeError("gguf_packed_bank: payload read failed or source changed")


class LoadCancelled(_lib.NativeError):
    """load_projections was cancelled; nothing was bound."""


def _check_cancel(cancel) -> None:
    if cancel is None:
        return
    hit = cancel.is_set() if hasattr(cancel, "is_set") else bool(cancel())
    if hit:
        raise LoadCancelled("gguf_packed_bank: load cancelled")


def _identity(path: str) -> tuple:
    st = os.stat(path)
    return (st.st_dev, st.st_ino, st.st_size, st.st_mtime_ns)


PAGER_ALIGN = 256  # byte alignment of each tensor inside a pager slot (tc_pager_create)


def _align(n: int) -> int:
    return -(-n // PAGER_ALIGN) * PAGER_ALIGN


class GGUFPager:
    """Streams groups of projections through a bounded set of device slots (tc_pager_*), the
    MI355X counterpart of the reference's GgufWeightPager fill / bind / retire
    (native/runtime/streaming/gguf_weight_pager.hpp:27-53) for models whose raw GGUF blocks do
    not all fit in device memory.

    ``groups``: one list of projection prefixes per group (for example one transformer block
    each); each prefix contributes its ``.weight`` and optional ``.bias`` tensors. With S slots,
    groups g + 1 .. g + S - 1 are read and uploaded while group g is in use; the upload of
    group g + S starts once g's reader fence has passed.

        with GGUFFile(path) as f, GGUFPager(f, [[f"blk.{i}.attn_q", f"blk.{i}.ffn_down"] for i in
                                                 range(n_blocks)], slot_count=3) as pager:
            for i, W in pager.iterate():
                y = W.project(x, f"blk.{i}.attn_q")

    A group's projections are bound (``qlinear.Weights``) over views of its slot, after the
    host has waited for the upload; the reader fence is recorded on the current stream (or
    ``stream``) when the caller moves to the next group, so work queued on that stream for
    the group finishes before its slot is overwritten."""

    def __init__(self, file: GGUFFile, groups, slot_count: int = 2):
        from . import qlinear as _ql
        self._ql = _ql
        self.file = file
        self.groups = [list(g) for g in groups]
        if not self.groups or slot_count < 1:
            raise _lib.NativeError("gguf_pager: no groups or no slots")
        self.slot_count = slot_count
        members, indices, begin = [], [], [0]
        for g in self.groups:
            ms = []
            for prefix in g:
                wname = file._find(prefix, ".weight")
                if wname is None:
                    raise _lib.NativeError(f"gguf_tensor_missing: {prefix}.weight")
                t = file.tensor(wname)
                if t.ggml_type not in gguf.TYPES or len(t.dims) != 2:
                    raise _lib.NativeError(f"{wname}: the device projection takes 2-D weights of a registered type")
                bname = file._find(prefix, ".bias")
                if bname is not None and file.tensor(bname).ggml_type not in _PLAIN:
                    raise _lib.NativeError(f"{bname}: not a plain F32/F16/BF16 tensor")
                ms.append((prefix, wname, bname))
                indices.append(file._index[wname])
                if bname is not None:
                    indices.append(file._index[bname])
            members.append(ms)
            begin.append(len(indices))
        self._members = members
        sizes = [sum(_align(file.tensors[i].bytes) for i in indices[begin[g]:begin[g + 1]])
                 for g in range(len(self.groups))]
        self.slot_bytes = max(max(sizes), PAGER_ALIGN)
        self._slots = [torch.empty(self.slot_bytes, dtype=torch.uint8, device="cuda") for _ in range(slot_count)]
        self._cancel = C.c_int(0)
        gb = (C.c_uint32 * len(begin))(*begin)
        ix = (C.c_uint64 * max(len(indices), 1))(*indices)
        sp = (C.c_void_p * slot_count)(*[t.data_ptr() for t in self._slots])
        h = C.c_void_p()
        _lib.call(_lib.lib().tc_pager_create, file._h, len(self.groups), gb, ix, slot_count, sp, self.slot_bytes,
                  C.byref(h))
        self._h = h
        self._offsets = []
        for g in range(len(self.groups)):
            n = begin[g + 1] - begin[g]
            offs, cnt, nbytes = (C.c_uint64 * max(n, 1))(), C.c_uint32(), C.c_uint64()
            _lib.call(_lib.lib().tc_pager_group_layout, self._h, g, offs, max(n, 1), C.byref(cnt), C.byref(nbytes))
            self._offsets.append(list(offs)[:cnt.value])

    # -- the fill / bind / retire steps
    def fill(self, group: int, slot: int) -> _lib.tc_pager_ticket:
        """Start reading `group` into `slot` (asynchronous); returns the slot's ticket."""
        t = _lib.tc_pager_ticket()
        _lib.call(_lib.lib().tc_pager_fill, self._h, group, slot, C.byref(self._cancel), C.byref(t))
        return t

    def bind(self, ticket) -> "object":
        """Wait for the ticket's upload, then bind its projections over views of the slot."""
        _lib.call(_lib.lib().tc_pager_acquire, self._h, C.byref(ticket), None)
        slot = self._slots[ticket.slot]
        offs = iter(self._offsets[ticket.group])
        W = self._ql.Weights()
        for prefix, wname, bname in self._members[ticket.group]:
            t = self.file.tensor(wname)
            o = next(offs)
            blocks = slot[o: o + t.bytes]
            bias = None
            if bname is not None:
                b = self.file.tensor(bname)
                ob = next(offs)
                bias = slot[ob: ob + b.bytes].view(_PLAIN[b.ggml_type]).reshape(-1)
                if bias.numel() != t.dims[1]:
                    raise _lib.NativeError(f"{bname}: {bias.numel()} values for {t.dims[1]} outputs")
            W.bind(canonical_name(prefix), blocks, t.ggml_type, t.dims[1], t.dims[0], bias)
        return W

    def retire(self, ticket, stream=None) -> None:
        """Record the reader fence of the ticket's slot on `stream` (default: the current one)."""
        s = (stream if stream is not None else torch.cuda.current_stream()).cuda_stream
        _lib.call(_lib.lib().tc_pager_release, self._h, C.byref(ticket), C.c_void_p(s))

    def iterate(self, stream=None):
        """Yield (group index, Weights) for every group in order, reading ahead into the other
        slots. A group's Weights are valid until the next group is requested: its slot is then
        retired (fence on `stream`, default the current stream) and refilled with a later group."""
        G, S = len(self.groups), self.slot_count
        tickets = {g: self.fill(g, g % S) for g in range(min(S, G))}
        for g in range(G):
            ticket = tickets.pop(g)
            W = self.bind(ticket)
            try:
                yield g, W
            finally:
                del W
                self.retire(ticket, stream)
            if g + S < G:
                tickets[g + S] = self.fill(g + S, g % S)

    def cancel(self) -> None:
        """Stop every fill in progress or queued at its next 4 MiB chunk (their bind raises
        NativeCancelled)."""
        self._cancel.value = 1

    def resume(self) -> None:
        """Clear a cancel() for the fills issued from now on."""
        self._cancel.value = 0

    def metrics(self) -> dict:
        m = _lib.tc_pager_metrics()
        _lib.lib().tc_pager_get_metrics(self._h, C.byref(m))
        return {"fills": m.fills, "bytes_read": m.bytes_read, "read_seconds": m.read_seconds,
                "wait_seconds": m.wait_seconds}

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            _lib.lib().tc_pager_free(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def validate_split(files: Iterable[GGUFFile]) -> None:
    """Split-set consistency (gguf_directory.hpp:269-304)."""
    fs = list(files)
    arr = (C.c_void_p * len(fs))(*[f._h.value for f in fs])
    _lib.call(_lib.lib().tc_gguf_validate_split, arr, len(fs))
