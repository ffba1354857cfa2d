"""TEST INFRASTRUCTURE ONLY -- CPU oracle for the GGUF Q4_K/Q6_K quantized-linear path.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may import
this module, and only as the checker or the timed CPU baseline; the product package
``turbocider_amd`` never imports it.

Byte/bit work (decode, conversions, quantizers) lives in ``tc_oracle.c`` (built into
``oracle/liboracle.so`` by ``oracle/Makefile``); this module wraps it with ctypes and adds
the numpy restatement of the quantized linear:

* ``linear_reference`` -- ``Weights::project`` quantized branch followed by runtime LoRA
  and bias (native/backends/mlx.cpp:626-722, 957-984): base GEMM with fp32-or-better
  accumulation cast once to bf16 (mlx.cpp:678-679), then per adapter, in order,
  ``y = bf16(f32(y) + f32(scale * f32(low @ B^T)))`` with ``low = f32(x @ A^T)``
  (mlx.cpp:702-704, 972-984), then the bias last, ``y = bf16(f32(y) + f32(bf16(bias)))``
  (mlx.cpp:687-688). Sums are taken in float64 and rounded once to float32, which is the
  fp32 result up to summation order.

* ``act_reference`` -- the output activations of a projection (tc_qlinear_forward_act):
  GELU in its tanh form (native/models/qwen21/transformer.cpp:48-57) and the gated
  ``silu(gate) * up`` (transformer.cpp:971-975, silu mlx.cpp:1627-1631), evaluated in float64
  on the projection's bf16 outputs and rounded once to bf16 (RNE).

Parity status per function: the activations are pinned by torch's float64 GELU / SiLU (an
independent implementation), odd-part identities and limits; decode / conversions are pinned by the reference-written
golden vectors and KATs; the LoRA/bias sequence by the fixed-bit KATs restated from
tests/native/native_lora_math_test.cpp; the GEMM by brute-force fp64 on small shapes and by
exact closed forms (one-hot activations); the quantizers are parity unpinned by design
(the reference has no quantizer) and pinned by properties.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libggufref.so"

TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K = 12, 13, 14
TYPE_F32, TYPE_F16, TYPE_BF16 = 0, 1, 30
TYPE_Q4_0, TYPE_Q4_1, TYPE_Q5_0, TYPE_Q5_1, TYPE_Q8_0 = 2, 3, 6, 7, 8
# Registered types (native/core/gguf_directory.hpp:21-26): bytes and elements per block.
BLOCK_BYTES = {TYPE_Q4_K: 144, TYPE_Q5_K: 176, TYPE_Q6_K: 210, TYPE_F32: 4, TYPE_F16: 2, TYPE_BF16: 2,
               TYPE_Q4_0: 18, TYPE_Q4_1: 20, TYPE_Q5_0: 22, TYPE_Q5_1: 24, TYPE_Q8_0: 34}
BLOCK_ELEMENTS = {t: 256 if t in (TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K) else 1 if t in (TYPE_F32, TYPE_F16, TYPE_BF16)
                  else 32 for t in BLOCK_BYTES}
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2

_lib = None
_ref = None


def build(ref: bool = False) -> None:
    """Compile the oracle (and, if asked and /root/reference exists, the reference decoder)."""
    targets = ["all"] + (["ref"] if ref and Path("/root/reference/native/core/gguf_decode.cpp").exists() else [])
    subprocess.run(["make", "-s", "-C", str(HERE), *targets], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        L.oracle_error.restype = C.c_char_p
        L.oracle_fp16_to_float.argtypes = [C.c_uint16]
        L.oracle_fp16_to_float.restype = C.c_float
        L.oracle_float_to_bf16_rne.argtypes = [C.c_float, C.POINTER(C.c_uint16)]
        L.oracle_float_to_fp16_rne.argtypes = [C.c_float, C.POINTER(C.c_uint16)]
        L.oracle_bf16_bits.argtypes = [C.c_float]
        L.oracle_bf16_bits.restype = C.c_uint16
        L.oracle_decode.argtypes = ([C.c_uint32, C.c_void_p] + [C.c_uint64] * 7 + [C.c_uint32, C.c_void_p]
                                    + [C.c_uint64] * 3 + [C.c_void_p, C.c_uint64, C.c_int, C.c_void_p])
        L.oracle_decode_rows_parallel.argtypes = [C.c_uint32, C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint32,
                                                  C.c_void_p, C.c_int]
        L.oracle_quantize.argtypes = [C.c_uint32, C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p]
        L.oracle_lora_apply_bf16.argtypes = ([C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p, C.c_uint64,
                                              C.c_uint64, C.c_uint64, C.c_void_p, C.c_void_p, C.c_uint32,
                                              C.c_float, C.c_uint64, C.c_uint64])
        L.oracle_bias_bf16.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_void_p]
        L.oracle_max_threads.restype = C.c_int
        _lib = L
    return _lib


def ref_lib() -> C.CDLL | None:
    """The reference's own decoder compiled into oracle/_ref (None when not built)."""
    global _ref
    if _ref is None and REF_PATH.exists():
        L = C.CDLL(str(REF_PATH))
        L.tcref_error.restype = C.c_char_p
        L.tcref_half.argtypes = [C.c_uint16]
        L.tcref_half.restype = C.c_float
        L.tcref_round.argtypes = [C.c_uint32, C.c_float, C.POINTER(C.c_uint16)]
        L.tcref_decode.argtypes = ([C.c_uint32, C.c_void_p] + [C.c_uint64] * 7 + [C.c_uint32, C.c_void_p]
                                   + [C.c_uint64] * 3 + [C.c_void_p, C.c_uint64, C.c_int, C.c_void_p])
        _ref = L
    return _ref


# ---------------------------------------------------------------------------------------
# scalar conversions (gguf_decode.cpp:377-405)
# ---------------------------------------------------------------------------------------
def fp16_to_float(bits: int) -> float:
    return lib().oracle_fp16_to_float(bits)


def round_bf16(value: float) -> tuple[int, int]:
    out = C.c_uint16()
    status = lib().oracle_float_to_bf16_rne(value, C.byref(out))
    return status, out.value


def round_fp16(value: float) -> tuple[int, int]:
    out = C.c_uint16()
    status = lib().oracle_float_to_fp16_rne(value, C.byref(out))
    return status, out.value


# ---------------------------------------------------------------------------------------
# decode (decode_cpu_into / decode_cpu_gather semantics)
# ---------------------------------------------------------------------------------------
def decode_raw(raw: bytes, typ: int, source_rows: int, source_columns: int, row_begin: int = 0,
               rows: int | None = None, column_begin: int = 0, columns: int | None = None, dtype: int = 0,
               row_stride: int | None = None, column_stride: int | None = None, gather=None,
               cancel: bool = False, target_size: int | None = None, fill: int = 0xA5, use_ref: bool = False):
    """Decode into a guard-filled byte target; returns (status, target bytes, receipt, error)."""
    L = ref_lib() if use_ref else lib()
    if L is None:
        raise RuntimeError("reference decoder not built (make -C oracle ref)")
    rows = source_rows if rows is None else rows
    if gather is not None:
        rows = len(gather)
    columns = source_columns - column_begin if columns is None else columns
    item = 4 if dtype == 0 else 2
    column_stride = item if column_stride is None else column_stride
    row_stride = columns * column_stride if row_stride is None else row_stride
    size = (rows - 1) * row_stride + columns * column_stride if target_size is None else target_size
    target = (C.c_ubyte * max(size, 1))(*([fill] * max(size, 1)))
    source = C.create_string_buffer(bytes(raw), len(raw))
    idx = (C.c_uint64 * len(gather))(*gather) if gather is not None else None
    stats = (C.c_uint64 * 5)()
    fn = L.tcref_decode if use_ref else L.oracle_decode
    status = fn(typ, source, len(raw), source_rows, source_columns, row_begin, rows, column_begin, columns,
                dtype, target, size, row_stride, column_stride, idx, len(gather) if gather is not None else 0,
                int(cancel), stats)
    err = (L.tcref_error() if use_ref else L.oracle_error()).decode()
    return status, bytes(target)[:size], list(stats), err


def decode_matrix(raw: np.ndarray, typ: int, rows: int, columns: int, dtype: int = DTYPE_F32,
                  threads: int | None = None) -> np.ndarray:
    """Dense row-major decode of a whole [rows, columns] K-quant tensor (row-parallel)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    assert raw.nbytes >= rows * columns // 256 * BLOCK_BYTES[typ]
    out = np.empty((rows, columns), dtype=np.float32 if dtype == DTYPE_F32 else np.uint16)
    status = lib().oracle_decode_rows_parallel(typ, raw.ctypes.data, rows, columns, dtype, out.ctypes.data,
                                               threads or os.cpu_count() or 1)
    if status:
        raise ValueError(lib().oracle_error().decode())
    return out


def quantize(typ: int, w: np.ndarray) -> np.ndarray:
    """Own K-quant quantizer (no reference counterpart): fp32 [rows, cols] -> raw block bytes."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    out = np.zeros(rows * cols // 256 * BLOCK_BYTES[typ], dtype=np.uint8)
    if lib().oracle_quantize(typ, w.ctypes.data, rows, cols, out.ctypes.data):
        raise ValueError(lib().oracle_error().decode())
    return out


# ---------------------------------------------------------------------------------------
# bf16 helpers (bit-exact RNE, gguf_decode.cpp:389-394 without the error path)
# ---------------------------------------------------------------------------------------
def bf16_bits(x: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_bits_from_f64(v: np.ndarray) -> np.ndarray:
    """float64 -> bf16 bits, round to nearest even (one rounding): the float64 value is first
    narrowed to float32 with round-to-odd (truncate, then set the last bit if inexact), which
    keeps the final RNE to bf16 exact since float32 carries 16 more bits."""
    v = np.asarray(v, dtype=np.float64)
    f = v.astype(np.float32)
    over = np.abs(f.astype(np.float64)) > np.abs(v)
    f = np.where(over, np.nextafter(f, np.float32(0)), f)
    bits = f.view(np.uint32).copy()
    inexact = (f.astype(np.float64) != v) & np.isfinite(v)
    bits |= inexact.astype(np.uint32)
    b = bits.astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def gelu_tanh_f64(z: np.ndarray) -> np.ndarray:
    """0.5 z (1 + tanh(u)), u = sqrt(2/pi) (z + 0.044715 z^3) (transformer.cpp:48-57), in float64
    as z / (1 + exp(-2u)): the same function (1 + tanh(u) = 2 / (1 + exp(-2u))), written so that
    it keeps full precision where 1 + tanh(u) cancels (z below about -5)."""
    z = np.asarray(z, dtype=np.float64)
    u = np.sqrt(2.0 / np.pi) * (z + 0.044715 * z ** 3)
    with np.errstate(over="ignore"):
        return z / (1.0 + np.exp(-2.0 * u))


def silu_f64(g: np.ndarray) -> np.ndarray:
    """g * sigmoid(g) in float64 (mlx.cpp:1627-1631)."""
    g = np.asarray(g, dtype=np.float64)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g))


ACT_NONE, ACT_GELU_TANH, ACT_SILU_GLU = 0, 1, 2


_PI = __import__("decimal").Decimal("3.14159265358979323846264338327950288419716939937510582097494")


def _near_bf16_tie(v: np.ndarray) -> np.ndarray:
    """Values whose float64 representation sits on or next to a bf16 rounding boundary, where
    the float64 evaluation error could decide the rounding."""
    f = v.astype(np.float32)
    low = f.view(np.uint32) & 0xFFFF
    return np.isfinite(v) & (v != 0) & ((low >= 0x7FFE) & (low <= 0x8002))


def _bf16_round_decimal(val, lo_bits: int) -> int:
    """RNE of a high-precision Decimal `val` to bf16, given the bf16 bits just below |val|."""
    from decimal import Decimal
    lo = Decimal(float(bf16_to_f32(np.array([lo_bits], np.uint16))[0]))
    hi = Decimal(float(bf16_to_f32(np.array([lo_bits + 1], np.uint16))[0]))
    a = abs(val)
    if a < lo or a > hi:
        raise ValueError("bf16 neighbours do not bracket the value")
    mid = (lo + hi) / 2
    up = a > mid or (a == mid and (lo_bits & 1))
    bits = lo_bits + 1 if up else lo_bits
    return bits | (0x8000 if val < 0 else 0)


def _refine(out: np.ndarray, v: np.ndarray, exact) -> np.ndarray:
    """Re-rounds the near-tie entries of `out` (bf16 of float64 `v`) from exact(i), a Decimal of
    60 significant digits: the oracle then rounds the exact value, not its float64 image."""
    from decimal import localcontext
    idx = np.flatnonzero(_near_bf16_tie(v).reshape(-1))
    if idx.size == 0:
        return out
    flat = out.reshape(-1)
    with localcontext() as ctx:
        ctx.prec = 60
        for i in idx:
            val = exact(int(i))
            trunc = int(np.abs(v.reshape(-1)[i:i + 1]).astype(np.float32).view(np.uint32)[0] >> 16)
            # The float32 image may sit just above the value: step down until lo <= |val|.
            for lo in (trunc, trunc - 1):
                try:
                    flat[i] = _bf16_round_decimal(val, lo)
                    break
                except ValueError:
                    continue
    return out


def act_reference(pre_bf16: np.ndarray, act: int) -> np.ndarray:
    """The output activation on finished bf16 projection outputs pre [m, n]: GELU per output,
    or silu(gate) * up per interleaved pair (columns 2c, 2c + 1 -> output column c), rounded
    once to bf16 from the exact value: float64 everywhere, and for values within reach of a
    bf16 rounding boundary (for instance g u exactly halfway between two bf16 values with
    sigmoid(g) = 1 in float64) a 60-digit decimal evaluation."""
    from decimal import Decimal
    z = bf16_to_f32(pre_bf16).astype(np.float64)
    if act == ACT_NONE:
        return np.asarray(pre_bf16, dtype=np.uint16).copy()
    if act == ACT_GELU_TANH:
        v = gelu_tanh_f64(z)
        flat = z.reshape(-1)

        def exact(i):
            d = Decimal(float(flat[i]))
            two_u = 2 * (2 / _PI).sqrt() * (d + Decimal("0.044715") * d ** 3)
            return d / (1 + (-two_u).exp())
        return _refine(bf16_bits_from_f64(v), v, exact)
    if act == ACT_SILU_GLU:
        g, u = z[..., 0::2], z[..., 1::2]
        v = silu_f64(g) * u
        gf, uf = g.reshape(-1), u.reshape(-1)

        def exact(i):
            dg, du = Decimal(float(gf[i])), Decimal(float(uf[i]))
            return dg * du / (1 + (-dg).exp())
        return _refine(bf16_bits_from_f64(v), v, exact)
    raise ValueError(f"unknown activation {act}")


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------------------------------
# quantized linear: base GEMM, runtime LoRA, bias (mlx.cpp:626-722, 957-984)
# ---------------------------------------------------------------------------------------
def gemm_f32(x_bf16: np.ndarray, w: np.ndarray) -> np.ndarray:
    """acc[M,N] = x @ w^T summed in float64 and rounded once to float32."""
    xf = bf16_to_f32(x_bf16).astype(np.float64)
    return (xf @ np.asarray(w, dtype=np.float64).T).astype(np.float32)


def lora_delta_f32(x_bf16: np.ndarray, a_bf16: np.ndarray, b_bf16: np.ndarray) -> np.ndarray:
    """delta = f32(f32(x @ A^T) @ B^T) (mlx.cpp:957-966 rank in fp32, :972-977 B product)."""
    low = (bf16_to_f32(x_bf16).astype(np.float64) @ bf16_to_f32(a_bf16).astype(np.float64).T).astype(np.float32)
    return (low.astype(np.float64) @ bf16_to_f32(b_bf16).astype(np.float64).T).astype(np.float32)


def apply_adapter(y_bf16: np.ndarray, x_bf16: np.ndarray, a_bf16, b_bf16, scale: float, row_begin: int = 0,
                  row_count: int | None = None, out_begin: int = 0, out_end: int | None = None) -> np.ndarray:
    """One adapter: y = bf16(f32(y) + f32(scale * delta)) on the selected rows/columns."""
    y = y_bf16.copy()
    row_count = y.shape[0] - row_begin if row_count is None else row_count
    out_end = y.shape[1] if out_end is None else out_end
    rows = slice(row_begin, row_begin + row_count)
    delta = lora_delta_f32(x_bf16[rows], a_bf16, b_bf16)
    t = np.float32(scale) * delta
    base = bf16_to_f32(y[rows, out_begin:out_end])
    y[rows, out_begin:out_end] = bf16_bits(base + t)
    return y


def add_bias(y_bf16: np.ndarray, bias_bf16: np.ndarray) -> np.ndarray:
    return bf16_bits(bf16_to_f32(y_bf16) + bf16_to_f32(bias_bf16)[None, :])


def bias_to_bf16(bias: np.ndarray | None, bias_dtype: str = "f32") -> np.ndarray | None:
    """astype(bias, bf16) (mlx.cpp:688): fp32 -> bf16 RNE; fp16 via fp32 (exact) then RNE."""
    if bias is None:
        return None
    if bias_dtype == "bf16":
        return np.asarray(bias, dtype=np.uint16)
    if bias_dtype == "f16":
        return bf16_bits(f16_bits_to_f32(bias))
    return bf16_bits(np.asarray(bias, dtype=np.float32))


def linear_reference(x_bf16: np.ndarray, w_decoded: np.ndarray, bias_bf16: np.ndarray | None = None,
                     adapters=()) -> np.ndarray:
    """Reference quantized linear on decoded weights (fp32 or bf16-as-fp32 values).

    adapters: iterable of dicts {a, b, scale, row_begin, row_count, out_begin, out_end}.
    """
    return linear_reference_chain(x_bf16, w_decoded, bias_bf16, adapters)[0]


def linear_reference_chain(x_bf16: np.ndarray, w_decoded: np.ndarray, bias_bf16: np.ndarray | None = None,
                           adapters=(), base_bf16: np.ndarray | None = None) -> tuple[np.ndarray, list]:
    """linear_reference, also returning its bf16 rounding chain: the values before the final
    rounding step, in order (the base projection, then after each adapter but the last step).
    ``base_bf16``: start from these base bits instead of computing the base GEMM (to check
    the adapters and the bias on top of a kernel's own base output)."""
    y = bf16_bits(gemm_f32(x_bf16, w_decoded)) if base_bf16 is None else np.asarray(base_bf16, dtype=np.uint16)
    chain = []
    for ad in adapters:
        chain.append(y)
        y = apply_adapter(y, x_bf16, ad["a"], ad["b"], ad["scale"], ad.get("row_begin", 0),
                          ad.get("row_count"), ad.get("out_begin", 0), ad.get("out_end"))
    if bias_bf16 is not None:
        chain.append(y)
        y = add_bias(y, bias_bf16)
    return y, chain


def lora_apply_scalar(x_bf16: np.ndarray, y_bf16: np.ndarray, a_bf16, b_bf16, scale: float, row_begin=0,
                      row_count=None, out_begin=0, out_end=None) -> np.ndarray:
    """Scalar C restatement (fp32 sums in index order) of native_lora_math_test.cpp:72-107."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    y = np.ascontiguousarray(y_bf16, dtype=np.uint16).copy()
    a = np.ascontiguousarray(a_bf16, dtype=np.uint16)
    b = np.ascontiguousarray(b_bf16, dtype=np.uint16)
    row_count = y.shape[0] - row_begin if row_count is None else row_count
    out_end = y.shape[1] if out_end is None else out_end
    lib().oracle_lora_apply_bf16(x.ctypes.data, x.shape[1], x.shape[1], y.ctypes.data, y.shape[1], row_begin,
                                 row_count, a.ctypes.data, b.ctypes.data, a.shape[0], scale, out_begin, out_end)
    return y


# ---------------------------------------------------------------------------------------
# comparison metrics used by the parity tests
# ---------------------------------------------------------------------------------------
def compare_bf16(actual: np.ndarray, expected: np.ndarray) -> dict:
    """rel-L2, max-abs, number of outputs differing by >= 1 bf16 ulp, and max error in ulps."""
    a = bf16_to_f32(actual).astype(np.float64)
    e = bf16_to_f32(expected).astype(np.float64)
    diff = np.abs(a - e)
    rel_l2 = float(np.sqrt((diff ** 2).sum() / max((e ** 2).sum(), 1e-30)))
    mag = np.maximum(np.abs(e), 2.0 ** -126)
    ulp = 2.0 ** (np.floor(np.log2(mag)) - 7)
    ulps = diff / ulp
    return {"rel_l2": rel_l2, "max_abs": float(diff.max(initial=0.0)), "flips": int((ulps >= 1).sum()),
            "max_ulps": float(ulps.max(initial=0.0)), "count": int(e.size)}


def _bf16_ulp(v: np.ndarray) -> np.ndarray:
    return 2.0 ** (np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126))) - 7)


FP32_UNIT = 2.0 ** -24


def abs_term_sum(x_bf16: np.ndarray, w: np.ndarray) -> np.ndarray:
    """S[m, n] = sum_k |x[m, k] * w[n, k]| (float64): the scale of the fp32 summation error of
    an output. Two correct fp32 evaluations of one dot product in different orders differ by a
    few units of FP32_UNIT * S, which exceeds a bf16 ulp only where the terms cancel to a
    result far smaller than S."""
    return np.abs(bf16_to_f32(x_bf16)).astype(np.float64) @ np.abs(np.asarray(w, dtype=np.float64)).T


def lora_abs_term_sum(x_bf16: np.ndarray, a_bf16: np.ndarray, b_bf16: np.ndarray, scale: float) -> np.ndarray:
    """Summation-error scale of one runtime adapter's delta: |s| (|x| |A|^T) |B|^T (float64)."""
    low = np.abs(bf16_to_f32(x_bf16)).astype(np.float64) @ np.abs(bf16_to_f32(a_bf16)).astype(np.float64).T
    return abs(float(scale)) * (low @ np.abs(bf16_to_f32(b_bf16)).astype(np.float64).T)


def _chain_magnitude(expected: np.ndarray, chain) -> np.ndarray:
    mag = np.abs(bf16_to_f32(expected).astype(np.float64))
    for c in chain:
        if c is not None:
            mag = np.maximum(mag, np.abs(bf16_to_f32(c).astype(np.float64)))
    return mag


def allowed_differing(count: int, fraction: float) -> int:
    """Outputs allowed to differ at all: `fraction` of them, plus a Poisson margin so that small
    output counts are not judged on a handful of rounding flips."""
    mean = fraction * count
    return int(mean + 3.0 * np.sqrt(mean) + 2)


def within_ulps(actual: np.ndarray, expected: np.ndarray, chain=(), term_sum: np.ndarray | None = None,
                c: float = 4.0, max_flip_fraction: float = 1e-3) -> tuple[bool, dict]:
    """Tight bound for a kernel whose only difference from the oracle is the order of its fp32
    sums (same decoded weights):

    * at most ``allowed_differing(count, max_flip_fraction)`` outputs differ at all, and
    * each output is within one bf16 ulp per rounding of its chain (``chain``: the oracle's
      intermediate bf16 values before the final rounding, e.g. the output before the bias),
      the ulp taken at the largest magnitude along the chain, plus ``c * FP32_UNIT *
      term_sum`` (the summation-order error of outputs whose terms cancel; see abs_term_sum).
      A rounding adds at most one ulp to a difference already present in its input: a one-ulp
      flip of y before the bias becomes two ulps of bf16(y + bias) when y + bias is a tie
      that the flip turns into the neighbouring tie, which rounds to even the other way.
    """
    a = bf16_to_f32(actual).astype(np.float64)
    e = bf16_to_f32(expected).astype(np.float64)
    diff = np.abs(a - e)
    ulp = _bf16_ulp(_chain_magnitude(expected, chain))
    bound = (1 + len(chain)) * ulp + (c * FP32_UNIT * term_sum if term_sum is not None else 0.0)
    differing = int((diff > 0).sum())
    allowed = allowed_differing(int(e.size), max_flip_fraction)
    excess = diff / bound
    info = {"differing": differing, "allowed": allowed, "count": int(e.size),
            "max_diff_over_bound": float(excess.max(initial=0.0))}
    if excess.size and excess.max() > 1.0:
        worst = int(np.argmax(excess))
        info["worst"] = {"actual": float(a.flat[worst]), "expected": float(e.flat[worst]),
                         "ulp": float(ulp.flat[worst]),
                         "term_sum": float(term_sum.flat[worst]) if term_sum is not None else None}
    return bool(excess.max(initial=0.0) <= 1.0 and differing <= allowed), info


def within_tolerance(stats: dict, actual: np.ndarray, expected: np.ndarray, rel_l2: float = 1e-2,
                     max_abs: float = 2e-2, chain=()) -> bool:
    """rel-L2 <= 1e-2 and max-abs <= 2e-2, where an output whose bf16 ulp
    (at the largest magnitude of its rounding chain) exceeds the absolute bound may instead
    differ by one ulp per bf16 rounding of the chain (1 + len(chain)): each rounding of a
    correctly computed value can flip once under a different fp32 summation order."""
    a = bf16_to_f32(actual).astype(np.float64)
    e = bf16_to_f32(expected).astype(np.float64)
    diff = np.abs(a - e)
    ulp = _bf16_ulp(_chain_magnitude(expected, chain))
    ok = (diff <= max_abs) | (diff <= (1 + len(chain)) * ulp)
    return bool(stats["rel_l2"] <= rel_l2 and ok.all())
