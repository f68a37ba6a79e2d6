"""Build libpragnosia_hip.so for gfx950 from pragnosia_amd/csrc/*.hip with hipcc (no JIT, no torch extension).

    python -m pragnosia_amd.build            # compile every source, link the library in-tree

The library lands next to this file, so it travels with the source tree. Objects go to pragnosia_amd/_build/.
Two measurement-only libraries are built beside it: libpragnosia_microbench.so (csrc/microbench/*.hip) and
libpragnosia_stamps.so (the scan kernels compiled with phase stamps, -DPRAGNOSIA_PHASE_STAMPS), both for bench.py.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libpragnosia_hip.so")
# measurement-only kernels (bench.py), kept out of the product library
MB_CSRC = os.path.join(CSRC, "microbench")
MB_LIB = os.path.join(HERE, "libpragnosia_microbench.so")
# the scan kernels with phase stamps (bench.py --phase-rates), kept out of the product library
STAMP_SRCS = [os.path.join(CSRC, f) for f in ("aspin_chunk.hip", "aspin_delta.hip")]
STAMP_LIB = os.path.join(HERE, "libpragnosia_stamps.so")
ARCH = "gfx950"

# -packed-fp32-ops off: packed fp32 forms are never generated (hipcc's host pass warns that the feature is unknown
# to it; that warning is harmless).
HIPFLAGS = ["--offload-arch=" + ARCH, "-O3", "-fPIC", "-std=c++17", "-ffp-contract=fast",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-result"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def sources(d: str = CSRC):
    return sorted(os.path.join(d, f) for f in os.listdir(d) if f.endswith(".hip"))


def _compile(src: str, verbose: bool, stamps: bool = False) -> str:
    sub = "st_" if stamps else ("mb_" if os.path.dirname(src) == MB_CSRC else "")
    obj = os.path.join(OBJ, sub + os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc(), *HIPFLAGS, *(["-DPRAGNOSIA_PHASE_STAMPS"] if stamps else []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    if verbose and r.stderr.strip():
        err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
        if err.strip():
            print(err, file=sys.stderr)
    return obj


def _link(objs, lib: str) -> None:
    tmp = lib + ".tmp"
    cmd = [hipcc(), "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every csrc/*.hip and link libpragnosia_hip.so; csrc/microbench/*.hip into libpragnosia_microbench.so
    and the scan kernels with phase stamps into libpragnosia_stamps.so (bench.py's measurement builds). Always
    recompiles. Returns the library path."""
    os.makedirs(OBJ, exist_ok=True)
    srcs, mb = sources(), sources(MB_CSRC)
    work = [(s, False) for s in srcs + mb] + [(s, True) for s in STAMP_SRCS]
    jobs = jobs or min(len(work), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda a: _compile(a[0], verbose, a[1]), work))
    n, m = len(srcs), len(srcs) + len(mb)
    _link(objs[:n], LIB)
    _link(objs[n:m], MB_LIB)
    _link(objs[m:], STAMP_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
