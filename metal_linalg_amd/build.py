"""Build libmetal_linalg.so for gfx950 with hipcc.

Every source under csrc/ is compiled as HIP (kernels and host code alike) for
the MI355X only, into objects under _build/, then linked into
metal_linalg_amd/libmetal_linalg.so, in-tree so that the GPU box loads the
same file.  Run as ``python -m metal_linalg_amd.build`` or through
``__graft_entry__.build()``.
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmetal_linalg.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # no packed-FP32 instructions (v_pk_*_f32) in any kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
    "-I", CSRC,
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unused-result",
]


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, "-x", "hip", "-c", src, "-o", obj] + FLAGS
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    if r.stderr.strip():
        # hipcc's host pass warns that it does not know the packed-fp32 feature
        lines = [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
        if lines:
            sys.stderr.write("\n".join(lines) + "\n")
    return obj


def _includes(path: str, seen: set) -> set:
    """path and the in-tree headers it includes, transitively."""
    if path in seen or not os.path.exists(path):
        return seen
    seen.add(path)
    with open(path) as f:
        for line in f:
            m = re.match(r'\s*#\s*include\s*[<"]([^>"]+)[>"]', line)
            if m:
                for d in (CSRC, os.path.join(ROOT, "include")):
                    _includes(os.path.join(d, m.group(1)), seen)
    return seen


def _stale(src: str) -> bool:
    """The object is missing or older than its source or a header it includes."""
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if not os.path.exists(obj):
        return True
    return os.path.getmtime(obj) < max(os.path.getmtime(d) for d in _includes(src, set()))


def build(jobs: int | None = None, incremental: bool = False) -> str:
    """Compile every source (or, with incremental, only the stale ones) and link."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    todo = [s for s in srcs if _stale(s)] if incremental else srcs
    jobs = jobs or max(1, min(8, len(todo), os.cpu_count() or 1))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_compile, todo))
    objs = [os.path.join(BUILD, os.path.basename(s) + ".o") for s in srcs]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp] + objs + ["-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(incremental="--incremental" in sys.argv))
