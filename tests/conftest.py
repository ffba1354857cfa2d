"""Shared test setup: the `gpu` marker, repository import path, golden fixtures."""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device); run with -m gpu")


@pytest.fixture(scope="session")
def golden():
    """(manifest, arrays) written by tests/golden/make_golden.py from the reference decoder."""
    manifest = json.loads((GOLDEN / "kquant_golden.json").read_text())
    with np.load(GOLDEN / "kquant_golden.npz", allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    return manifest, arrays


@pytest.fixture(scope="session")
def other_golden():
    """(manifest, arrays) of the F32 / F16 / BF16 and legacy-block decode cases
    (tests/golden/make_golden.py, main_other)."""
    manifest = json.loads((GOLDEN / "other_golden.json").read_text())
    with np.load(GOLDEN / "other_golden.npz", allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    return manifest, arrays


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle
    oracle.build()
    return oracle


@pytest.fixture
def ref_decoder():
    """The reference's own decoder built into oracle/_ref (checker only). Probed inside the
    test that needs it, never at collection, so that processes which do not run such a test
    (the GPU suite) never load it; skips where it is not built (no /root/reference)."""
    from oracle import oracle
    lib = oracle.ref_lib()
    if lib is None:
        pytest.skip("reference decoder not built (needs /root/reference)")
    return lib
