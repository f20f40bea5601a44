"""Builds libmegamoe.so for gfx950 with hipcc, in-tree, next to this file.

The build also keeps the compiler's per-kernel resource report (VGPRs, spills, scratch,
occupancy) in libmegamoe.kernels.json beside the library: a kernel that starts to spill runs
slower with no change in its results, so the tests read the report.
"""

from __future__ import annotations

import json
import os
import re
import subprocess
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO = PACKAGE_DIR.parent
SOURCE = PACKAGE_DIR / "csrc" / "megamoe.hip"
OUTPUT = PACKAGE_DIR / "libmegamoe.so"
REPORT = PACKAGE_DIR / "libmegamoe.kernels.json"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # Rounding points are written explicitly; no implicit fused multiply-add.
    "-ffp-contract=off",
    # No packed fp32 VALU instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Per-kernel register, spill and scratch figures (remarks on stderr).
    "-Rpass-analysis=kernel-resource-usage",
]

_FIELDS = {
    "VGPRs": "vgprs", "AGPRs": "agprs", "SGPRs": "sgprs", "ScratchSize [bytes/lane]": "scratch_bytes",
    "Occupancy [waves/SIMD]": "occupancy", "SGPRs Spill": "sgpr_spills", "VGPRs Spill": "vgpr_spills",
    "LDS Size [bytes/block]": "lds_bytes",
}


def resource_report(stderr: str) -> dict:
    """{mangled function name: {field: int}} from hipcc's kernel-resource-usage remarks."""
    out: dict = {}
    name = None
    for line in stderr.splitlines():
        m = re.search(r"remark:\s+(.*?):\s+(\S+)\s+\[-Rpass-analysis=kernel-resource-usage\]", line)
        if not m:
            continue
        key, value = m.group(1).strip(), m.group(2)
        if key == "Function Name":
            name = value
            out[name] = {}
        elif name is not None and key in _FIELDS:
            out[name][_FIELDS[key]] = int(value)
    return out


def build_library(verbose: bool = False, defines: tuple[str, ...] = (), output: Path | None = None) -> Path:
    """Builds the library (``output``: another path, for a check build with ``defines``, e.g.
    ``MEGAMOE_AGENT_ACQUIRE=1``; its resource report is not kept)."""
    out = OUTPUT if output is None else Path(output)
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, *[f"-D{d}" for d in defines], f"-I{REPO / 'include'}", str(SOURCE), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stderr}")
    other = [l for l in proc.stderr.splitlines() if "kernel-resource-usage" not in l]
    if verbose and any(l.strip() for l in other):
        print("\n".join(other))
    report = resource_report(proc.stderr)
    if not report:
        raise RuntimeError("hipcc printed no kernel resource report")
    if output is None:
        REPORT.write_text(json.dumps(report, indent=1, sort_keys=True) + "\n")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("-D", dest="defines", action="append", default=[], help="a macro for hipcc, NAME=VALUE")
    ap.add_argument("-o", dest="output", default=None, help="library path (default: the in-tree libmegamoe.so)")
    args = ap.parse_args()
    print(build_library(verbose=True, defines=tuple(args.defines), output=args.output))
