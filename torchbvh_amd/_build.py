"""Build the native library (``libtorchbvh_amd.so``) in-tree with hipcc.

The library is a plain C-ABI shared object (no torch headers, no Python C
API), compiled for gfx950 only.  ``python -m torchbvh_amd._build`` rebuilds it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR / "csrc"
LIB_NAME = "libtorchbvh_amd.so"
LIB_PATH = PACKAGE_DIR / LIB_NAME
SOURCES = ("build.hip", "sort.hip", "small.hip", "accel.hip", "knn.hip", "route.hip", "interp.hip", "capi.hip")
ARCH = "gfx950"


def hipcc_path() -> str:
    found = shutil.which("hipcc")
    if found:
        return found
    candidate = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc"
    if candidate.exists():
        return str(candidate)
    raise RuntimeError("hipcc not found; the torchbvh_amd native library needs ROCm")


def compile_command(output: Path = LIB_PATH) -> list[str]:
    return [
        hipcc_path(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # Deterministic fp32: IEEE division, explicit FMAs only.
        "-ffp-contract=off",
        "-fno-fast-math",
        # Packed fp32 VALU ops stay off on this target.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-function",
        "-o", str(output),
        *[str(CSRC / s) for s in SOURCES],
    ]


def build(verbose: bool = False) -> Path:
    """Compile the native library into the package directory; return its path."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = compile_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            "hipcc failed building torchbvh_amd:\n" + proc.stdout + proc.stderr
        )
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
