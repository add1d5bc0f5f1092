"""Build step of the HIP library: hipcc for gfx950 -> libmvme_paged.so (in-tree).

The reference JIT-builds its CUDA extension on first use
(mini_engine/kernels/cuda_extension.py:14-66).  This package instead builds
one plain C-ABI shared object ahead of time so that the same file travels with
the source tree and is loaded with ctypes; nothing is compiled at import time.

Run ``python -m mini_engine_hip.build`` (with the package directory on
``sys.path``) or call :func:`build_library`.
"""

from __future__ import annotations

import concurrent.futures
import hashlib
import os
from pathlib import Path
import shutil
import subprocess
import sys

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR.parent / "csrc"
INCLUDE_DIR = PACKAGE_DIR.parents[1] / "include"
LIB_DIR = PACKAGE_DIR / "_lib"
LIB_NAME = "libmvme_paged.so"
ARCH = "gfx950"

# Packed-FP32 VALU forms are disabled for every HIP translation unit; hipcc's
# host pass warns that it does not know the feature, which is harmless.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def library_path() -> Path:
    return LIB_DIR / LIB_NAME


def digest_path() -> Path:
    return LIB_DIR / "SOURCE_DIGEST"


def sources() -> list[Path]:
    return sorted(SOURCE_DIR.glob("*.hip"))


def source_digest() -> str:
    digest = hashlib.sha256()
    for path in sorted([*SOURCE_DIR.glob("*.hip"), *SOURCE_DIR.glob("*.h"), *INCLUDE_DIR.glob("*.h")]):
        digest.update(path.name.encode())
        digest.update(path.read_bytes())
    return digest.hexdigest()


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    if candidate.exists():
        return str(candidate)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: the HIP library cannot be built")
    return found


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(cmd)}\n{result.stderr}")


def build_library(*, jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libmvme_paged.so.

    Always recompiles (the build check must exercise the compiler).  The
    source digest is written next to the library; the loader refuses a
    library whose digest differs from the current sources.
    """
    hipcc = _hipcc()
    build_dir = PACKAGE_DIR / "_build"
    build_dir.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    objects = []
    commands = []
    for src in sources():
        obj = build_dir / (src.stem + ".o")
        objects.append(obj)
        commands.append([hipcc, *HIP_FLAGS, f"-I{INCLUDE_DIR}", "-c", str(src), "-o", str(obj)])
    workers = jobs or min(len(commands), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        for cmd, _ in zip(commands, pool.map(_run, commands)):
            if verbose:
                print(" ".join(cmd), flush=True)
    target = library_path()
    tmp = target.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)])
    os.replace(tmp, target)
    digest_path().write_text(source_digest() + "\n")
    return target


if __name__ == "__main__":
    path = build_library(verbose="-v" in sys.argv)
    print(path)
