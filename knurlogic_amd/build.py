"""Build libknurlogic_amd.so from csrc/*.hip with hipcc for gfx950 (in tree)."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "csrc"
OUT = HERE / "libknurlogic_amd.so"
ARCH = os.environ.get("KMI_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    # packed fp32 ops stay off: hipcc would otherwise form them from scalar code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def sources():
    return sorted(SRC.glob("*.hip"))


def build(verbose: bool = False) -> Path:
    """Compile every HIP source into one shared library; always rebuilds."""
    tmp = OUT.with_suffix(".so.tmp")
    cmd = ["hipcc", *FLAGS, *map(str, sources()), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
