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


# Per-source flags: MFMA results in VGPRs where VALU code consumes them --
# the skinny kernels' per-group scale FMAs, and the KV8 kernels' softmax
# rescale of O -- which would otherwise copy them out of AGPRs first
# (MoE 16 tokens 67.5 -> 64.9 us, 256 tokens 153.6 -> 148.2; KV8 64 rows at
# D = 512 97.4 -> 80.2; the GEMMs and the VQ kernels measured even or slower
# with it, and keep their accumulators in AGPRs).
EXTRA = {f: ["-mllvm", "-amdgpu-mfma-vgpr-form"] for f in ("qgemv.hip", "qgemv_xs.hip", "qgemv_dl.hip", "kv8.hip")}


# The compiler's per-kernel resource remarks (registers, scratch, occupancy),
# parsed after each compile.
RESOURCE_REMARKS = "-Rpass-analysis=kernel-resource-usage"

# Kernels that stage through direct-to-LDS loads wait for them with counted
# `s_waitcnt vmcnt(N)`: N counts the vector-memory operations the wave issued
# after the stage's loads, which holds only while nothing else -- a register
# spill's scratch store or load above all -- sits among them.  Every kernel
# compiled from a source (or a local header it includes) that names one of
# these must use no scratch.
DMA_MARKERS = ("buffer_load_lds", "wait_vmcnt<")


def sources():
    return sorted(SRC.glob("*.hip"))


def uses_lds_dma(src: Path) -> bool:
    """Whether src, or a csrc header it includes, issues direct-to-LDS loads
    or counted vmcnt waits."""
    texts = [src.read_text()]
    for line in texts[0].splitlines():
        line = line.strip()
        if line.startswith("#include \"") and line.endswith(".hpp\""):
            h = SRC / line.split("\"")[1]
            if h.exists():
                texts.append(h.read_text())
    return any(m in t for t in texts for m in DMA_MARKERS)


def kernel_scratch(remarks: str) -> dict:
    """{mangled kernel name: scratch bytes per lane} from the resource remarks."""
    out, name = {}, None
    for line in remarks.splitlines():
        if "remark: Function Name: " in line:
            name = line.split("remark: Function Name: ")[1].split()[0]
        elif "ScratchSize [bytes/lane]: " in line and name is not None:
            out[name] = int(line.split("ScratchSize [bytes/lane]: ")[1].split()[0])
    return out


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (r.stderr or "").splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    return err


def _drop_remarks(text: str) -> str:
    """The compiler output without the resource remarks and the source
    excerpts ("  157 | ...", "      | ^") clang prints under each."""
    out, skip = [], False
    for line in text.splitlines():
        if "kernel-resource-usage" in line:
            skip = True
            continue
        if skip and line.lstrip()[:1] in ("|",) or (skip and line.strip().split(" |")[0].isdigit()):
            continue
        skip = False
        out.append(line)
    return "\n".join(out)


def check_scratch(src: Path, remarks: str) -> dict:
    """The scratch each kernel of src uses; raises when a kernel of a
    direct-to-LDS source spills (its counted waits would no longer count
    only its stage loads)."""
    sc = kernel_scratch(remarks)
    if uses_lds_dma(src):
        bad = {k: v for k, v in sc.items() if v}
        if bad:
            raise RuntimeError(f"{src.name}: kernels with direct-to-LDS loads and counted vmcnt waits use "
                               f"scratch (a spill breaks the waits' count): {bad}")
    return sc


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
        errs = list(ex.map(lambda so: _run(["hipcc", *cflags, *EXTRA.get(so[0].name, []), RESOURCE_REMARKS,
                                            "-c", str(so[0]), "-o", str(so[1])]),
                           zip(srcs, objs)))
    spills = {}
    for src, e in zip(srcs, errs):
        spills.update({k: v for k, v in check_scratch(src, e).items() if v})
    errs = [_drop_remarks(e) for e in errs]
    if verbose and spills:
        print("kernels using scratch (bytes per lane): " + ", ".join(f"{k} {v}" for k, v in sorted(spills.items())),
              file=sys.stderr)
    tmp = OUT.with_suffix(".so.tmp")
    errs.append(_run(["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC",
                      *map(str, objs), "-o", str(tmp)]))
    if verbose and any(e.strip() for e in errs):
        print("\n".join(e for e in errs if e.strip()), file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
