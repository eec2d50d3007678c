"""Build libhkx.so, the gfx950 kernels and their C ABI, in-tree.

    python hk-dsl_amd/build.py            # -> hk-dsl_amd/hk/_lib/libhkx.so

Each translation unit under csrc/ is compiled by hipcc for gfx950 in parallel and
linked into one shared library. The build refuses a kernel that spills (scratch
memory per lane > 0), read from the compiler's resource-usage remarks -- the
equivalent of the reference's spill gate (python/hk/runtime/resources.py:1-40).
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
OUT = HERE / "hk" / "_lib"
LIB = OUT / "libhkx.so"
PROBE_SRC = HERE / "probes" / "peaks.hip"
PROBE_LIB = OUT / "libhkx_probe.so"
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
    # Packed fp32 VALU ops are kept out of the code: the compiler would otherwise
    # form v_pk_* from ordinary float code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Rpass-analysis=kernel-resource-usage",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _compile(src: Path, obj: Path) -> str:
    cmd = [hipcc(), *FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr[-4000:]}")
    return r.stderr


def _spills(remarks: str) -> list:
    """Kernels whose remarks report scratch memory, as (name, bytes)."""
    out, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name and int(m.group(1)) > 0:
            out.append((name, int(m.group(1))))
    return out


def build(verbose: bool = False, jobs: int = 8) -> Path:
    OUT.mkdir(parents=True, exist_ok=True)
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [objdir / (s.stem + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        remarks = list(ex.map(_compile, srcs, objs))
    bad = [sp for r in remarks for sp in _spills(r)]
    if bad:
        raise RuntimeError("kernels spill to scratch memory: "
                           + ", ".join(f"{n} ({b} B/lane)" for n, b in bad))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    # the measured-ceilings probe (bench.py reports roofline fractions against it too)
    r = subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-O3", "-shared", "-fPIC",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                        "-o", str(PROBE_LIB), str(PROBE_SRC)], capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"probe build failed:\n{r.stderr[-4000:]}")
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True, jobs=int(os.environ.get("MAX_JOBS", "8")))
