"""Builds libmegamoe.so for gfx950 with hipcc, in-tree, next to this file."""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO = PACKAGE_DIR.parent
SOURCE = PACKAGE_DIR / "csrc" / "megamoe.hip"
OUTPUT = PACKAGE_DIR / "libmegamoe.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # Rounding points are written explicitly; no implicit fused multiply-add.
    "-ffp-contract=off",
    # No packed fp32 VALU instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def build_library(verbose: bool = False) -> Path:
    tmp = OUTPUT.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, f"-I{REPO / 'include'}", str(SOURCE), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stderr}")
    if verbose and proc.stderr.strip():
        print(proc.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build_library(verbose=True))
