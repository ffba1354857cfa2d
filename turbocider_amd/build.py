"""Build the HIP library ``turbocider_amd/libtc_qlinear.so`` for gfx950 with hipcc.

Every kernel source under ``csrc/`` is compiled to an object in ``turbocider_amd/_build/``
(in parallel; the GEMM kernel source once per variant, see ``VARIANTS``) and linked into one
shared library that exports the C ABI declared in
``include/tc_qlinear.h``. The library is built in-tree so that it travels with the
repository snapshot to the GPU machine.

    python -m turbocider_amd.build          # or: python turbocider_amd/build.py
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libtc_qlinear.so"
ARCH = os.environ.get("TC_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    # Keep the compiler from emitting packed fp32 (v_pk_*_f32) instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the turbocider_amd HIP library cannot be built")
    return path


# Sources compiled once per variant (-D definitions), so that the variants build in parallel.
VARIANTS = {
    "k_gemm_variant": [
        (f"{t}_{s}_{mt}_{a}", [f"-DTC_GEMM_TYPE={t}", f"-DTC_GEMM_SPLIT={s}", f"-DTC_GEMM_MT={mt}",
                               f"-DTC_GEMM_ACT={a}"])
        for t in (12, 13, 14) for s in (0, 1) for mt in (1, 2, 4, 8)
        for a in (((0, 1, 2, 3) if mt >= 4 else (0, 1, 2)) if s == 0 else (0,))
    ] + [
        # Grouped launches (two problems in one work list): 128- and 256-row tiles only.
        (f"g{t}_{s}_{mt}", [f"-DTC_GEMM_TYPE={t}", f"-DTC_GEMM_SPLIT={s}", f"-DTC_GEMM_MT={mt}", "-DTC_GEMM_ACT=0",
                            "-DTC_GEMM_GROUP=1"])
        for t in (12, 13, 14) for s in (0, 1) for mt in (4, 8)
    ],
}


def _units(sources):
    """(source, object suffix, extra flags) for every object to build."""
    for src in sources:
        for suffix, defs in VARIANTS.get(src.stem, [("", [])]):
            yield src, suffix, defs


def _compile(unit, incremental: bool = False) -> Path:
    src, suffix, defs = unit
    obj = BUILD / (src.stem + (f"_{suffix}" if suffix else "") + ".o")
    if incremental and obj.exists():
        newest = max(p.stat().st_mtime for p in [src, *CSRC.glob("*.h")])
        if obj.stat().st_mtime > newest:
            return obj
    cmd = [hipcc(), *HIPCC_FLAGS, *defs, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False, incremental: bool = False) -> Path:
    """Compile every source (or, with ``incremental``, only those newer than their object)
    and link the library."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    units = list(_units(sources))
    # Largest compile units first, so that they do not finish last on a loaded pool.
    units.sort(key=lambda u: (u[0].stem != "k_gemm_variant", u[1].endswith("_8") is False))
    jobs = min(len(units), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(lambda u: _compile(u, incremental), units))
    tmp = LIB.with_suffix(".so.tmp")
    rocm_lib = Path(hipcc()).resolve().parents[1] / "lib"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp),
           f"-L{rocm_lib}", f"-Wl,-rpath,{rocm_lib}", "-lrocblas"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv[1:])
