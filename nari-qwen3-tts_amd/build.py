"""Build recipe for the in-tree HIP library ``libnq_hip.so`` (gfx950 only).

Each ``csrc/*.hip`` file compiles to its own object with hipcc and the objects
link into one shared library that exports the C ABI of ``include/nq_abi.h``.
Translation units whose results must be bit-identical to the oracle (the
sampler) are built with ``-ffp-contract=off``.  Nothing here runs a GPU: hipcc
cross-compiles for gfx950 on any host.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR / "csrc"
LIBRARY = PACKAGE_DIR / "libnq_hip.so"
MEASURE_LIBRARY = PACKAGE_DIR / "libnq_measure.so"
OBJ_DIR = PACKAGE_DIR / "_build"
ARCH = "gfx950"

# Packed-FP32 instructions stay disabled in every device pass.
_COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]
_EXACT_FP = {"nq_sampler.hip"}


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


def _compile(hipcc: str, source: Path) -> Path:
    obj = OBJ_DIR / (source.stem + ".o")
    flags = list(_COMMON)
    if source.name in _EXACT_FP:
        flags.append("-ffp-contract=off")
    cmd = [hipcc, *flags, "-c", str(source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build_library(verbose: bool = False) -> Path:
    """Compile every kernel source and link ``libnq_hip.so`` in the package."""

    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError("no HIP sources under csrc/")
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objects = list(pool.map(lambda s: _compile(hipcc, s), sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(sources)} sources")
    _build_measure(hipcc, verbose)
    return LIBRARY


def _build_measure(hipcc: str, verbose: bool) -> None:
    """The benchmark's measurement kernels (``csrc/measure``) as their own library,
    ``libnq_measure.so``, outside the serving library and its ABI."""

    sources = sorted((CSRC / "measure").glob("*.hip"))
    if not sources:
        return
    tmp = MEASURE_LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc, *_COMMON, "-shared", "-o", str(tmp), *map(str, sources)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"measurement library build failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, MEASURE_LIBRARY)
    if verbose:
        print(f"built {MEASURE_LIBRARY}")


if __name__ == "__main__":
    build_library(verbose=True)
