"""CPU: kernel routing and activation-layout guards of tc_qlinear_forward, through the C ABI's
host-only tc_qlinear_plan (the same planning code forward runs; no device needed).

The kernels address activations with 32-bit buffer offsets. A row stride so large that one
output tile's rows do not fit those offsets must be rejected before any launch, and a very
tall activation (a span from a tile's first row to row M of 4 GiB or more) must still route
to the GEMM, whose descriptor range is clamped rather than wrapped.
"""
from __future__ import annotations

import ctypes as C

import pytest

from turbocider_amd import _lib

Q4K, Q6K, Q8_0 = 12, 14, 8
GEMM, GEMV1, GEMV8, SKINNY, GEMV, DENSE = 1, 2, 3, 4, 5, 6


def plan(typ, n, k, m, x_stride=None, path=0):
    info = _lib.tc_qlinear_plan_info()
    msg = C.c_void_p()
    st = _lib.lib().tc_qlinear_plan(typ, n, k, m, k if x_stride is None else x_stride, path, C.byref(info),
                                    C.byref(msg))
    text = C.cast(msg, C.c_char_p).value.decode() if msg.value else ""
    if msg.value:
        _lib.lib().tc_qlinear_string_free(msg)
    return st, info, text


@pytest.mark.parametrize("typ", [Q4K, Q6K])
@pytest.mark.parametrize("m,kernel", [(1, GEMV1), (2, GEMV8), (8, GEMV8), (9, SKINNY), (64, SKINNY),
                                      (65, GEMM), (4096, GEMM)])
def test_routes_by_rows(typ, m, kernel):
    st, info, text = plan(typ, 3072, 3072, m)
    assert st == 0, text
    assert info.kernel == kernel


def test_forced_paths():
    assert plan(Q4K, 3072, 3072, 1, path=1)[1].kernel == GEMM
    assert plan(Q4K, 3072, 3072, 5, path=2)[1].kernel == GEMV
    assert plan(Q4K, 3072, 3072, 40, path=3)[1].kernel == SKINNY
    st, _, text = plan(Q4K, 3072, 3072, 9, path=2)
    assert st == 1 and "at most 8 rows" in text
    st, _, text = plan(Q4K, 3072, 3072, 9, path=4)
    assert st == 1 and text == "invalid path"


def test_dense_types_route_to_library_gemm():
    st, info, _ = plan(Q8_0, 3072, 3072, 1024)
    assert st == 0 and info.kernel == DENSE and info.workspace_bytes == 0


def test_ltx_tail_rows_on_skinny_kernel():
    """4132 LTX tokens: 16 full 256-row tiles and a 36-row tail that would need a grid round
    of its own (256 CUs) run as GEMM + skinny tail."""
    st, info, text = plan(Q4K, 4096, 4096, 4132)
    assert st == 0, text
    assert info.kernel == GEMM and info.tail_rows == 36


def test_split_k_workspace_reported():
    st, info, _ = plan(Q4K, 3584, 3584, 256)   # 28 tiles of 128 rows: K split
    assert st == 0 and info.kernel == GEMM and info.workspace_bytes > 0
    st, info, _ = plan(Q4K, 12288, 3072, 4096)  # north star: 768 tiles, no split
    assert st == 0 and info.workspace_bytes == 0


def test_tall_activation_routes_to_gemm():
    """2^21 rows of K = 3072 (12 GiB of activations): every tile descriptor's span from its
    first row reaches past 4 GiB for the first tiles; accepted (range clamped in the kernel)."""
    st, info, text = plan(Q4K, 3072, 3072, 1 << 21)
    assert st == 0, text
    assert info.kernel == GEMM


@pytest.mark.parametrize("m", [100, 1 << 20])
def test_huge_row_stride_rejected_on_gemm(m):
    """A row stride of 2^23 elements: 255 rows from a tile's first row exceed 2^31 bytes."""
    st, _, text = plan(Q4K, 3072, 3072, m, x_stride=1 << 23)
    assert st == 1
    assert "32-bit offsets" in text


def test_largest_accepted_row_stride():
    limit = ((1 << 31) // 2 - 3072 - 1) // 255
    assert plan(Q4K, 3072, 3072, 300, x_stride=limit)[0] == 0
    assert plan(Q4K, 3072, 3072, 300, x_stride=limit + 1)[0] == 1


def test_small_m_with_huge_stride_falls_back_then_rejects():
    """2..8 and 9..64 rows whose activation span exceeds the small-M kernels' 32-bit offsets
    leave those kernels; the GEMM then rejects the stride."""
    for m in (4, 40):
        st, _, text = plan(Q6K, 3584, 3584, m, x_stride=1 << 29)
        assert st == 1 and "32-bit offsets" in text
    st, info, _ = plan(Q6K, 3584, 3584, 4, x_stride=1 << 28)   # 2 (3 * 2^28 + K) < 2^31: still GEMV8
    assert st == 0 and info.kernel == GEMV8


def test_invalid_geometry():
    assert plan(Q4K, 3072, 3000, 4)[0] == 1
    assert plan(Q4K, 3072, 3072, 0)[0] == 1
    assert plan(Q4K, 3072, 3072, 4, x_stride=3000)[0] == 1
    assert plan(99, 3072, 3072, 4)[0] == 1


@pytest.mark.parametrize("m,kernel", [(1, GEMV1), (2, GEMV8), (8, GEMV8), (9, SKINNY), (40, SKINNY), (64, SKINNY),
                                      (65, GEMM), (4096, GEMM)])
def test_q5k_routes(m, kernel):
    """Q5_K runs the same hand-written kernels as Q4_K / Q6_K: the one-row GEMV at M = 1, the
    2..8-row GEMV, the skinny kernel at 9..64 rows, the MFMA dequant-GEMM above; never the
    library GEMM."""
    st, info, text = plan(13, 3072, 3072, m)
    assert st == 0, text
    assert info.kernel == kernel


def test_q5k_forced_per_row_gemv_rejected():
    st, _, text = plan(13, 512, 512, 3, path=2)
    assert st == 1 and "per-row GEMV takes Q4_K / Q6_K" in text
    st, info, _ = plan(13, 512, 512, 1, path=2)
    assert st == 0 and info.kernel == GEMV1
