"""Build recipe of the gfx950 kernel library ``libslc_hip.so``.

Every ``csrc/*.hip`` file is compiled with ``hipcc --offload-arch=gfx950`` into
an object under ``_build/`` and the objects are linked into one shared library
next to this file.  The library exports only the ``extern "C"`` entry points
declared in ``include/slc_hip.h``.  Runs on a CPU-only machine (hipcc
cross-compiles the device code).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parents[1]
CSRC = PACKAGE_DIR / "csrc"
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = REPO_ROOT / "_build"
LIBRARY = PACKAGE_DIR / "libslc_hip.so"
ARCH = os.environ.get("SLC_HIP_ARCH", "gfx950")

# -packed-fp32-ops: packed fp32 VALU forms are kept out of every kernel.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the HIP backend cannot be built")
    return found


def _compile(source: Path) -> Path:
    obj = BUILD_DIR / (source.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(
            f"hipcc failed for {source.name}:\n{result.stdout}\n{result.stderr}"
        )
    return obj


def build(verbose: bool = False) -> Path:
    """Compile all kernels and link ``libslc_hip.so``; returns its path."""

    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, (os.cpu_count() or 4)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [
        _hipcc(),
        f"--offload-arch={ARCH}",
        "-shared",
        "-fPIC",
        *map(str, objects),
        "-o",
        str(tmp),
    ]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stdout}\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
