"""Build libmambaqc_hip.so, the C-ABI library of HIP kernels, in-tree.

    python -m mambaqc_amd.build          # or mambaqc_amd.build.build()

Every ``csrc/*.hip`` file is compiled for gfx950 with hipcc (in parallel) and
linked into ``mambaqc_amd/lib/libmambaqc_hip.so``. Nothing is cached: each call
recompiles, so a stale library can never survive a source change.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
LIBNAME = "libmambaqc_hip.so"
ARCH = os.environ.get("MQC_OFFLOAD_ARCH", "gfx950")

# Packed fp32 VALU instructions are disabled for all device code (the compiler
# is otherwise free to emit them from float2-shaped arithmetic).
HIPFLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm under /opt/rocm")


# The compiler reports each kernel's register and scratch use as remarks.
RESOURCE_REMARKS = "-Rpass-analysis=kernel-resource-usage"
_FN = re.compile(r"remark: Function Name: (\S+)")
_SCRATCH = re.compile(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)")
_QUOTED = re.compile(r"^\s*(\d+\s*)?\|")  # source lines quoted under a remark


def _spilling_kernels(stderr: str) -> list[str]:
    """Kernels whose resource remarks show scratch memory (register spills)."""
    out, name = [], None
    for line in stderr.splitlines():
        m = _FN.search(line)
        if m:
            name = m.group(1)
            continue
        m = _SCRATCH.search(line)
        if m and name is not None and int(m.group(1)) > 0:
            out.append(f"{name} ({m.group(1)} bytes/lane)")
    return out


def _compile(hipcc: str, src: Path, obj: Path) -> None:
    cmd = [hipcc, *HIPFLAGS, RESOURCE_REMARKS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature and says so; that
    # warning is expected and filtered from the log, as are the resource
    # remarks (and the source lines the compiler quotes under them).
    noise = "'-packed-fp32-ops' is not a recognized feature"
    lines, includes, in_remark = [], [], False
    for l in r.stderr.splitlines():
        if noise in l:
            continue
        if l.startswith("In file included from"):
            includes.append(l)
            continue
        if "[-Rpass-analysis=kernel-resource-usage]" in l:
            includes, in_remark = [], True
            continue
        if in_remark and _QUOTED.match(l):
            continue
        in_remark = False
        lines += includes + [l]
        includes = []
    err = "\n".join(lines + includes)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    # Every kernel here is written to run from registers; scratch means a
    # launch shape or template instance outgrew its register budget.
    spills = _spilling_kernels(r.stderr)
    if spills:
        raise RuntimeError(f"{src.name}: kernels spill registers to scratch:\n  " +
                           "\n  ".join(spills))


def build(verbose: bool = True) -> Path:
    hipcc = _hipcc()
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [objdir / (s.stem + ".o") for s in sources]
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda so: _compile(hipcc, *so), zip(sources, objs)))
    out = LIBDIR / LIBNAME
    tmp = LIBDIR / (LIBNAME + ".tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} from {len(sources)} sources", file=sys.stderr)
    return out


if __name__ == "__main__":
    build()
