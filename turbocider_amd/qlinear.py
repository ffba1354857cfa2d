"""Quantized linear operator (GGUF weights: Q4_K / Q5_K / Q6_K fused, other types dense; bf16
activations) with runtime LoRA.

Mirrors the reference's operator interface on this path:

* ``Weights.project(x, prefix)`` -- ``tc::Weights::project`` (native/backends/mlx.hpp:203,
  mlx.cpp:626-690): ``<prefix>.weight`` (raw GGUF blocks), optional ``<prefix>.bias``,
  runtime LoRA terms bound to the prefix, applied in binding order, bias last.
* ``Weights.bind_runtime_lora`` -- the inference-time binding of ``apply_loras``
  (mlx.cpp:1437-1460,1502-1510): effective scale ``strength * alpha / rank`` when an alpha
  is present (else ``strength``), optional output row range for fused targets.
* ``QuantizedLinear`` -- one bound projection (a ``tc_qlinear`` handle).

Every call runs on the GPU through ``libtc_qlinear.so``; there is no CPU path.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .gguf import TYPES, row_bytes

PATH_AUTO, PATH_GEMM, PATH_GEMV = 0, 1, 2

# Output activations of tc_qlinear_forward_act (TC_QLINEAR_ACT_*).
ACTIVATIONS = {None: 0, "none": 0, "gelu_tanh": 1, "silu_glu": 2}

_BIAS_DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


class QLinearError(ValueError):
    """Rejected projection (the reference raises std::invalid_argument via require)."""


def lora_scale(strength: float, rank: int, alpha: float | None = None) -> float:
    """Effective runtime-LoRA scale, in the reference's fp32 steps (mlx.cpp:1442-1452):
    ``float scale = strength; scale *= alpha / float(rank);`` with ``strength`` a float
    (``LoRAAsset::strength``, core/contracts.hpp:17) and ``alpha`` read as float32. Every
    operation rounds to fp32: ``s = f32(s * f32(f32(alpha) / f32(rank)))``."""
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        scale = np.float32(strength)
        if alpha is not None:
            a = np.float32(alpha)
            if not math.isfinite(float(a)):
                raise QLinearError("LoRA alpha must be finite")
            scale = np.float32(scale * np.float32(a / np.float32(rank)))
    if not math.isfinite(float(scale)):
        raise QLinearError("LoRA effective scale must be finite")
    return float(scale)


@dataclass
class LoRAAdapter:
    """One runtime adapter: A ("down"/lora_A) [rank, K] and B ("up"/lora_B) [out_end-out_begin, rank]."""
    down: torch.Tensor
    up: torch.Tensor
    scale: float
    row_begin: int = 0
    row_count: int | None = None
    output_begin: int = 0
    output_end: int | None = None

    @property
    def rank(self) -> int:
        return int(self.down.shape[0])


def _stream(stream) -> int:
    return int((stream if stream is not None else torch.cuda.current_stream()).cuda_stream)


class QuantizedLinear:
    """y = x * deq(W)^T (+ runtime LoRA) (+ bias) for raw GGUF weights of shape [n, k]: Q4_K / Q5_K / Q6_K
    on the fused dequant kernels, any other registered type decoded once to bf16 and multiplied by
    the library GEMM (the reference's dense branch, native/backends/mlx.cpp:680-686)."""

    def __init__(self, weight_blocks: torch.Tensor, ggml_type: int, n: int, k: int,
                 bias: torch.Tensor | None = None):
        if ggml_type not in TYPES:
            raise QLinearError(f"gguf_type_unsupported: {ggml_type}")
        if weight_blocks.dtype != torch.uint8 or not weight_blocks.is_cuda or not weight_blocks.is_contiguous():
            raise QLinearError("weights must be a contiguous uint8 device tensor of raw GGUF blocks")
        if weight_blocks.numel() < n * row_bytes(ggml_type, k):
            raise QLinearError("weight buffer too short")
        if bias is not None and (bias.dtype not in _BIAS_DTYPE or bias.numel() != n or not bias.is_contiguous()):
            raise QLinearError("bias must be a contiguous [n] fp32/fp16/bf16 device tensor")
        self.weight, self.type, self.n, self.k, self.bias = weight_blocks, ggml_type, n, k, bias
        desc = _lib.tc_qlinear_desc(ggml_type, n, k, weight_blocks.data_ptr(), weight_blocks.numel(),
                                    bias.data_ptr() if bias is not None else None,
                                    _BIAS_DTYPE[bias.dtype] if bias is not None else 0)
        handle = C.c_void_p()
        try:
            _lib.call(_lib.lib().tc_qlinear_create, C.byref(desc), C.byref(handle))
        except _lib.NativeError as e:
            raise QLinearError(str(e)) from None
        self._handle = handle

    def set_path(self, path: int) -> None:
        _lib.call(_lib.lib().tc_qlinear_set_path, self._handle, path)

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h is not None and h.value:
            try:
                _lib.lib().tc_qlinear_free(h)
            except Exception:
                pass
            self._handle = None

    def forward(self, x: torch.Tensor, adapters=(), out: torch.Tensor | None = None, stream=None,
                allocation_free: bool = False, act: str | None = None) -> torch.Tensor:
        """x: [..., k] bf16 device tensor -> [..., n] bf16. ``allocation_free`` calls
        tc_qlinear_forward_noalloc (no device allocation inside the call; pass ``out`` too so
        that this method allocates nothing either). ``act``: output activation applied in the
        kernels' epilogue (tc_qlinear_forward_act): "gelu_tanh", or "silu_glu" for weights
        whose rows hold gate and up interleaved (glu_pair_rows; the output is n/2 wide)."""
        if act not in ACTIVATIONS:
            raise QLinearError(f"unknown output activation: {act}")
        code = ACTIVATIONS[act]
        if code and allocation_free:
            raise QLinearError("the allocation-free entry point applies no output activation")
        if x.dtype != torch.bfloat16 or not x.is_cuda or x.shape[-1] != self.k:
            raise QLinearError(f"input must be a bf16 device tensor with last dimension {self.k}")
        if code == 2 and self.n % 2:
            raise QLinearError("the gated activation needs an even number of outputs")
        width = self.n // 2 if code == 2 else self.n
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.k)
        if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
            x2 = x2.contiguous()
        m = x2.shape[0]
        y = out if out is not None else torch.empty((m, width), dtype=torch.bfloat16, device=x.device)
        if y.dtype != torch.bfloat16 or y.shape != (m, width) or y.stride(-1) != 1:
            raise QLinearError(f"output must be a bf16 [m, {width}] tensor with unit column stride")
        arr = (_lib.tc_lora_adapter * max(len(adapters), 1))()
        keep = []
        for i, ad in enumerate(adapters):
            a, b = ad.down.contiguous(), ad.up.contiguous()
            keep += [a, b]
            oe = self.n if ad.output_end is None else ad.output_end
            rc = m - ad.row_begin if ad.row_count is None else ad.row_count
            if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
                raise QLinearError("LoRA factors must be bf16")
            if a.shape != (ad.rank, self.k) or b.shape != (oe - ad.output_begin, ad.rank):
                raise QLinearError("invalid LoRA rank geometry")
            arr[i] = _lib.tc_lora_adapter(a.data_ptr(), b.data_ptr(), ad.rank, ad.scale, ad.row_begin, rc,
                                          ad.output_begin, oe)
        try:
            if code:
                _lib.call(_lib.lib().tc_qlinear_forward_act, self._handle, code, x2.data_ptr(), m, x2.stride(0),
                          y.data_ptr(), y.stride(0), arr, len(adapters), _stream(stream))
            else:
                entry = _lib.lib().tc_qlinear_forward_noalloc if allocation_free else _lib.lib().tc_qlinear_forward
                _lib.call(entry, self._handle, x2.data_ptr(), m, x2.stride(0), y.data_ptr(), y.stride(0), arr,
                          len(adapters), _stream(stream))
        except _lib.NativeError as e:
            raise QLinearError(str(e)) from None
        return y.reshape(*lead, width)

    __call__ = forward


def glu_pair_rows(gate_blocks: torch.Tensor, up_blocks: torch.Tensor, ggml_type: int, n: int, k: int) -> torch.Tensor:
    """Raw GGUF rows of a gate [n, k] and an up [n, k] weight interleaved into one [2n, k]
    weight, row 2c = gate row c and row 2c + 1 = up row c: the layout the gated activation
    ("silu_glu") reads, so that each output's gate and up land side by side in the epilogue.
    The bytes are copied unchanged (the decode of every row is the same)."""
    rb = row_bytes(ggml_type, k)
    for t in (gate_blocks, up_blocks):
        if t.dtype != torch.uint8 or not t.is_cuda or t.numel() < n * rb:
            raise QLinearError("gate and up must be uint8 device tensors of n rows of raw GGUF blocks")
    g = gate_blocks.reshape(-1)[: n * rb].view(n, rb)
    u = up_blocks.reshape(-1)[: n * rb].view(n, rb)
    return torch.stack((g, u), dim=1).reshape(-1).contiguous()


def glu_pair_bias(gate_bias: torch.Tensor | None, up_bias: torch.Tensor | None, n: int,
                  device) -> torch.Tensor | None:
    """The biases of a gate / up pair in glu_pair_rows order (a missing one is zeros)."""
    if gate_bias is None and up_bias is None:
        return None
    ref = gate_bias if gate_bias is not None else up_bias
    gb = gate_bias if gate_bias is not None else torch.zeros(n, dtype=ref.dtype, device=device)
    ub = up_bias if up_bias is not None else torch.zeros(n, dtype=ref.dtype, device=device)
    if gb.dtype != ub.dtype or gb.numel() != n or ub.numel() != n:
        raise QLinearError("gate and up biases must be [n] tensors of one dtype")
    return torch.stack((gb.reshape(-1), ub.reshape(-1)), dim=1).reshape(-1).contiguous()


def _glu_adapter(ad: LoRAAdapter, n: int) -> LoRAAdapter:
    """An adapter bound to a gate_up projection in the reference's column order (gate columns
    0..n-1, then up columns n..2n-1) re-expressed on the interleaved rows: B's row for column c
    moves to 2c (gate) or 2(c - n) + 1 (up) inside the adapter's new contiguous output span,
    and the span's other rows are zero (they add exactly zero to their outputs)."""
    ob, oe = ad.output_begin, (2 * n if ad.output_end is None else ad.output_end)
    cols = torch.arange(ob, oe, device=ad.up.device)
    dest = torch.where(cols < n, 2 * cols, 2 * (cols - n) + 1)
    lo, hi = int(dest.min()), int(dest.max()) + 1
    b = torch.zeros((hi - lo, ad.rank), dtype=ad.up.dtype, device=ad.up.device)
    b[dest - lo] = ad.up
    return LoRAAdapter(ad.down, b, ad.scale, ad.row_begin, ad.row_count, lo, hi)


def forward_many(linears, x: torch.Tensor, outs=None, stream=None) -> list:
    """Projections of one activation (no runtime LoRA): [lin(x) for lin in linears], as one
    fused launch for up to 8 rows (tc_qlinear_forward_many; Weights::project_many,
    mlx.cpp:724-760)."""
    linears = list(linears)
    if not linears:
        raise QLinearError("cannot project an empty prefix list")
    k = linears[0].k
    if x.dtype != torch.bfloat16 or not x.is_cuda or x.shape[-1] != k or any(l.k != k for l in linears):
        raise QLinearError(f"input must be a bf16 device tensor with last dimension {k} shared by all projections")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    ys = list(outs) if outs is not None else [torch.empty((m, l.n), dtype=torch.bfloat16, device=x.device)
                                               for l in linears]
    for y, l in zip(ys, linears):
        if y.dtype != torch.bfloat16 or y.shape != (m, l.n) or y.stride(-1) != 1:
            raise QLinearError("output must be a bf16 [m, n] tensor with unit column stride")
    n = len(linears)
    hs = (C.c_void_p * n)(*[l._handle for l in linears])
    yp = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
    st = (C.c_uint64 * n)(*[y.stride(0) for y in ys])
    try:
        _lib.call(_lib.lib().tc_qlinear_forward_many, hs, n, x2.data_ptr(), m, x2.stride(0), yp, st, _stream(stream))
    except _lib.NativeError as e:
        raise QLinearError(str(e)) from None
    return [y.reshape(*lead, l.n) for y, l in zip(ys, linears)]


def forward_group(linears, xs, outs=None, stream=None, act=None) -> tuple[list, bool]:
    """Projections of different activations (no runtime LoRA): [act(lin(x)) for lin, x in
    zip(linears, xs)] for one or two projections, as ONE grouped dequant-GEMM launch over the
    output tiles of both when they share weight type, k and activation row stride and each
    would run the GEMM on its own (tc_qlinear_forward_group: the image and text streams of a
    dual-stream block, flux_transformer.cpp:995-1004). `act` as QuantizedLinear.forward
    ("silu_glu": outputs n / 2 wide). Returns (outputs, grouped)."""
    linears, xs = list(linears), list(xs)
    if not linears or len(linears) != len(xs):
        raise QLinearError("forward_group needs one activation per projection")
    if act not in ACTIVATIONS:
        raise QLinearError(f"unknown output activation: {act}")
    code = ACTIVATIONS[act]
    if code == 2 and any(l.n % 2 for l in linears):
        raise QLinearError("the gated activation needs an even number of outputs")
    x2s, ys = [], []
    for i, (l, x) in enumerate(zip(linears, xs)):
        if x.dtype != torch.bfloat16 or not x.is_cuda or x.shape[-1] != l.k:
            raise QLinearError(f"input must be a bf16 device tensor with last dimension {l.k}")
        x2 = x.reshape(-1, l.k)
        if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
            x2 = x2.contiguous()
        x2s.append(x2)
        m = x2.shape[0]
        width = l.n // 2 if code == 2 else l.n
        y = outs[i] if outs is not None else torch.empty((m, width), dtype=torch.bfloat16, device=x.device)
        if y.dtype != torch.bfloat16 or y.shape != (m, width) or y.stride(-1) != 1:
            raise QLinearError("output must be a bf16 [m, width] tensor with unit column stride")
        ys.append(y)
    n = len(linears)
    hs = (C.c_void_p * n)(*[l._handle for l in linears])
    xp = (C.c_void_p * n)(*[x.data_ptr() for x in x2s])
    ms = (C.c_uint64 * n)(*[x.shape[0] for x in x2s])
    xst = (C.c_uint64 * n)(*[x.stride(0) for x in x2s])
    yp = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
    yst = (C.c_uint64 * n)(*[y.stride(0) for y in ys])
    grouped = C.c_uint32(0)
    try:
        _lib.call(_lib.lib().tc_qlinear_forward_group, hs, n, code, xp, ms, xst, yp, yst, _stream(stream),
                  C.byref(grouped))
    except _lib.NativeError as e:
        raise QLinearError(str(e)) from None
    return [y.reshape(*x.shape[:-1], y.shape[-1]) for y, x in zip(ys, xs)], bool(grouped.value)


class Weights:
    """Named quantized projections with runtime LoRA, like the reference's Weights dictionary."""

    def __init__(self):
        self._linears: dict[str, QuantizedLinear] = {}
        self._runtime: dict[str, list[LoRAAdapter]] = {}
        self._glu: dict[str, int] = {}  # gate_up prefixes bound with interleaved rows -> n
        self._stacks: dict[str, list[tuple[str, int, int]]] = {}  # stacked name -> (member, row0, n)

    def bind(self, prefix: str, weight_blocks: torch.Tensor, ggml_type: int, n: int, k: int,
             bias: torch.Tensor | None = None) -> QuantizedLinear:
        lin = QuantizedLinear(weight_blocks, ggml_type, n, k, bias)
        self._linears[prefix] = lin
        return lin

    def bind_glu(self, prefix: str, gate_blocks: torch.Tensor, up_blocks: torch.Tensor, ggml_type: int, n: int,
                 k: int, gate_bias: torch.Tensor | None = None, up_bias: torch.Tensor | None = None) -> QuantizedLinear:
        """Bind a gate [n, k] / up [n, k] pair as one gate_up projection (rows interleaved by
        glu_pair_rows). project() of it returns the reference's [gate; up] column order;
        project_act(..., "silu_glu") returns silu(gate) * up from the epilogue."""
        rows = glu_pair_rows(gate_blocks, up_blocks, ggml_type, n, k)
        bias = glu_pair_bias(gate_bias, up_bias, n, rows.device)
        lin = self.bind(prefix, rows, ggml_type, 2 * n, k, bias)
        self._glu[prefix] = n
        return lin

    def bind_gate_up(self, prefix: str, blocks: torch.Tensor, ggml_type: int, two_n: int, k: int,
                     bias: torch.Tensor | None = None) -> QuantizedLinear:
        """Bind a fused gate_up weight stored as [gate; up] ([2n, k], gate rows first: the
        reference's ``img_mlp.gate_up``, native/models/qwen21/transformer.cpp:971-975)."""
        if two_n % 2:
            raise QLinearError("a gate_up weight needs an even number of rows")
        n, rb = two_n // 2, row_bytes(ggml_type, k)
        flat = blocks.reshape(-1)
        if flat.numel() < two_n * rb:
            raise QLinearError("weight buffer too short")
        gb = ub = None
        if bias is not None:
            if bias.numel() != two_n:
                raise QLinearError("bias must be a [2n] tensor")
            gb, ub = bias.reshape(-1)[:n], bias.reshape(-1)[n:]
        return self.bind_glu(prefix, flat[: n * rb], flat[n * rb: two_n * rb], ggml_type, n, k, gb, ub)

    def bind_stacked(self, name: str, prefixes) -> QuantizedLinear:
        """Stack bound projections of one type and input width (each with a bias, or none with
        one) into a single projection `name` over their rows in order: projections that read
        the same activation then run as one launch (project_stacked), such as the adaLN
        modulation of every block of a DiT from one timestep embedding
        (native/models/qwen21/transformer.cpp:617; one 6-hidden modulation per block and stream
        in an MMDiT). The members are rebound as views of the stacked rows, so project(member)
        keeps working and no weight byte is held twice."""
        prefixes = list(prefixes)
        if not prefixes or len(set(prefixes)) != len(prefixes):
            raise QLinearError("a stack needs distinct member prefixes")
        if name in self._linears:
            raise QLinearError(f"projection already bound: {name}")
        for p in prefixes:
            if p not in self._linears:
                raise QLinearError(f"missing weight: {p}.weight")
            if p in self._glu or p in self._stacks:
                raise QLinearError(f"{p}: gate_up and stacked bindings cannot be stacked")
        lins = [self._linears[p] for p in prefixes]
        typ, k = lins[0].type, lins[0].k
        if any(l.type != typ or l.k != k for l in lins):
            raise QLinearError("stacked projections must share the weight type and input width")
        with_bias = [l.bias is not None for l in lins]
        if any(with_bias) and not all(with_bias):
            raise QLinearError("stacked projections must all have a bias or none")
        rb = row_bytes(typ, k)
        rows = torch.cat([l.weight.reshape(-1)[: l.n * rb] for l in lins])
        bias = torch.cat([l.bias.reshape(-1).float() for l in lins]) if all(with_bias) else None
        total = sum(l.n for l in lins)
        big = QuantizedLinear(rows, typ, total, k, bias)
        members, row0 = [], 0
        for p, l in zip(prefixes, lins):
            view = rows[row0 * rb: (row0 + l.n) * rb]
            self._linears[p] = QuantizedLinear(view, typ, l.n, k, l.bias)
            members.append((p, row0, l.n))
            row0 += l.n
        self._linears[name] = big
        self._stacks[name] = members
        return big

    def project_stacked(self, x: torch.Tensor, name: str, stream=None) -> dict:
        """All members of a stack from one launch: {member: its [..., n] output} (column views
        of one [..., total] output). Runtime adapters bound to the members apply to their
        columns."""
        if name not in self._stacks:
            raise QLinearError(f"not a stacked projection: {name}")
        ads = []
        for p, row0, n in self._stacks[name]:
            for ad in self._runtime.get(p, ()):
                oe = n if ad.output_end is None else ad.output_end
                ads.append(LoRAAdapter(ad.down, ad.up, ad.scale, ad.row_begin, ad.row_count,
                                       row0 + ad.output_begin, row0 + oe))
        y = self._linears[name].forward(x, ads, stream=stream)
        return {p: y[..., row0: row0 + n] for p, row0, n in self._stacks[name]}

    def has(self, prefix: str) -> bool:
        return prefix in self._linears

    def bound_prefixes(self) -> list[str]:
        return sorted(self._linears)

    def publish(self, linears: dict) -> None:
        """Bind a set of already-validated projections in one step (no prefix may be bound yet)."""
        clash = sorted(set(linears) & set(self._linears))
        if clash:
            raise QLinearError(f"projection already bound: {clash[0]}")
        self._linears.update(linears)

    def bind_runtime_lora(self, prefix: str, down: torch.Tensor, up: torch.Tensor, strength: float,
                          alpha: float | None = None, output_start: int = 0, output_end: int | None = None) -> None:
        """Bind one adapter to a projection (inference-time apply_loras, mlx.cpp:1437-1460,1502-1510)."""
        if prefix not in self._linears:
            raise QLinearError(f"LoRA target missing: {prefix}")
        if prefix in self._stacks:
            raise QLinearError(f"{prefix}: bind runtime adapters to the stack's members")
        lin = self._linears[prefix]
        if down.dim() != 2 or up.dim() != 2 or down.shape[0] != up.shape[1]:
            raise QLinearError(f"invalid LoRA rank geometry: {prefix}")
        if down.shape[1] != lin.k:
            raise QLinearError(f"LoRA input does not match {prefix}")
        end = lin.n if output_end is None else output_end
        if not (0 <= output_start < end <= lin.n) or up.shape[0] != end - output_start:
            raise QLinearError(f"invalid runtime LoRA output range: {prefix}")
        ad = LoRAAdapter(down.to(torch.bfloat16).contiguous(), up.to(torch.bfloat16).contiguous(),
                         lora_scale(strength, down.shape[0], alpha), 0, None, output_start, end)
        if prefix in self._glu:
            ad = _glu_adapter(ad, self._glu[prefix])
        self._runtime.setdefault(prefix, []).append(ad)

    def clear_runtime_loras(self) -> None:
        self._runtime.clear()

    def project(self, x: torch.Tensor, prefix: str, stream=None) -> torch.Tensor:
        if prefix not in self._linears:
            raise QLinearError(f"missing weight: {prefix}.weight")
        y = self._linears[prefix].forward(x, self._runtime.get(prefix, ()), stream=stream)
        if prefix in self._glu:
            # Interleaved gate/up rows back to the reference's [gate; up] column order.
            n = self._glu[prefix]
            y = y.reshape(*y.shape[:-1], n, 2).transpose(-1, -2).reshape(*y.shape[:-1], 2 * n)
        return y

    def project_act(self, x: torch.Tensor, prefix: str, act: str, stream=None) -> torch.Tensor:
        """act(project(x, prefix)) with the activation in the kernels' epilogue: "gelu_tanh",
        or "silu_glu" for a prefix bound by bind_glu / bind_gate_up (silu(gate) * up, n wide)."""
        if prefix not in self._linears:
            raise QLinearError(f"missing weight: {prefix}.weight")
        if (act == "silu_glu") != (prefix in self._glu):
            raise QLinearError(f"{prefix}: the gated activation needs a gate_up binding (bind_glu / bind_gate_up)"
                               if act == "silu_glu" else f"{prefix}: a gate_up binding takes the gated activation")
        return self._linears[prefix].forward(x, self._runtime.get(prefix, ()), stream=stream, act=act)

    def project_mlp(self, x: torch.Tensor, up_prefix: str, down_prefix: str, act: str | None = None,
                    stream=None) -> torch.Tensor:
        """down(act(up(x))): the feed-forward of a block (native/models/qwen21/transformer.cpp:
        969-978 with a gate_up binding and "silu_glu"; the GELU MLP of an MMDiT block with
        "gelu_tanh"). The activation runs in the up projection's epilogue, so the
        pre-activation outputs never go to memory; act defaults to "silu_glu" for a gate_up
        binding and "gelu_tanh" otherwise."""
        if act is None:
            act = "silu_glu" if up_prefix in self._glu else "gelu_tanh"
        h = self.project_act(x, up_prefix, act, stream=stream)
        return self.project(h, down_prefix, stream=stream)

    def project_many(self, x: torch.Tensor, prefixes, stream=None) -> list:
        """Projections of one activation (Weights::project_many, mlx.cpp:724-760): fused when
        no runtime LoRA is bound to any of them, else one project() per prefix."""
        prefixes = list(prefixes)
        if not prefixes:
            raise QLinearError("cannot project an empty prefix list")
        for p in prefixes:
            if p not in self._linears:
                raise QLinearError(f"missing weight: {p}.weight")
        if any(self._runtime.get(p) for p in prefixes):
            return [self.project(x, p, stream=stream) for p in prefixes]
        return forward_many([self._linears[p] for p in prefixes], x, stream=stream)

    def project_group(self, pairs, stream=None, act=None) -> list:
        """Projections of different activations, [(x, prefix), ...] of one or two entries (the
        image and text streams of a dual-stream block, flux_transformer.cpp:995-1004), with an
        optional output activation as project_act ("silu_glu" for gate_up bindings): one
        grouped launch (forward_group) when no runtime LoRA is bound to them; else one
        project() / project_act() each. Without an activation, gate_up bindings (interleaved
        rows, reordered by project()) also run one by one."""
        pairs = list(pairs)
        for _, p in pairs:
            if p not in self._linears:
                raise QLinearError(f"missing weight: {p}.weight")
            if act is not None and act != "none" and (act == "silu_glu") != (p in self._glu):
                raise QLinearError(f"{p}: the gated activation needs a gate_up binding (bind_glu / bind_gate_up)"
                                   if act == "silu_glu" else f"{p}: a gate_up binding takes the gated activation")
        plain = act is None or act == "none"
        if any(self._runtime.get(p) for _, p in pairs) or (plain and any(p in self._glu for _, p in pairs)):
            if plain:
                return [self.project(x, p, stream=stream) for x, p in pairs]
            return [self.project_act(x, p, act, stream=stream) for x, p in pairs]
        ys, _ = forward_group([self._linears[p] for _, p in pairs], [x for x, _ in pairs], stream=stream, act=act)
        return ys
