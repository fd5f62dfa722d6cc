"""Compile the C oracle (test infrastructure) into oracle/_build/liboracle.so.

gcc only; -ffp-contract=off keeps every fused multiply-add explicit (fmaf),
so the oracle's distance arithmetic is exactly the documented chain.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
BUILD_DIR = ORACLE_DIR / "_build"
LIB_PATH = BUILD_DIR / "liboracle.so"


def compile_command(output: Path) -> list[str]:
    return [
        os.environ.get("CC", "gcc"),
        "-O2",
        "-std=c11",
        "-fPIC",
        "-shared",
        "-fopenmp",
        "-ffp-contract=off",
        "-fno-fast-math",
        "-Wall",
        "-o",
        str(output),
        str(ORACLE_DIR / "oracle.c"),
        "-lm",
    ]


def build(verbose: bool = False) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = compile_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("gcc failed building the oracle:\n" + proc.stdout + proc.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
