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


# Per-source flags.  qgemv: MFMA results in VGPRs (the FMAs that consume them
# each group would otherwise copy them out of AGPRs first).
EXTRA = {"qgemv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def sources():
    return sorted(SRC.glob("*.hip"))


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (r.stderr or "").splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build(verbose: bool = False, jobs: int = 8) -> Path:
    """Compile every HIP source (in parallel, objects under _build/) and link
    one shared library; always rebuilds."""
    from concurrent.futures import ThreadPoolExecutor
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    cflags = [f for f in FLAGS if f != "-shared"]
    srcs = sources()
    objs = [objdir / (p.stem + ".o") for p in srcs]
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        errs = list(ex.map(lambda so: _run(["hipcc", *cflags, *EXTRA.get(so[0].name, []), "-c", str(so[0]),
                                            "-o", str(so[1])]),
                           zip(srcs, objs)))
    tmp = OUT.with_suffix(".so.tmp")
    errs.append(_run(["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC",
                      *map(str, objs), "-o", str(tmp)]))
    if verbose and any(e.strip() for e in errs):
        print("\n".join(e for e in errs if e.strip()), file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
