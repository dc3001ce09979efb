"""Build the gfx950 HIP library ``kanjoos_amd/libkanjoos_amd.so`` in-tree.

``python -m kanjoos_amd.build`` (or ``__graft_entry__.build()``) compiles every
``csrc/*.hip`` with hipcc for gfx950 and links one shared library exposing the C
ABI of ``include/knj_capi.h``.  Objects go to ``kanjoos_amd/_build/``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libkanjoos_amd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # no packed-FP32 instructions anywhere in this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    "-I", os.path.join(ROOT, "include"),
]


HOST = os.path.join(HERE, "host")
RUN = os.path.join(HERE, "kanjoos-run")


def sources():
    """HIP device+host sources, then the plain C++ host classes (compiled by
    hipcc as host code)."""
    hip = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    return hip + [os.path.join(HOST, f) for f in ("knj_host.cpp", "knj_profiler.cpp", "knj_residency.cpp")]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    if src.endswith(".cpp"):
        cmd = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-Wall", "-I", os.path.join(ROOT, "include"),
               "-c", src, "-o", obj]
    else:
        cmd = [HIPCC, *HIP_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    # the host pass warns about the unknown packed-fp32 feature; show only real warnings
    warn = [l for l in r.stderr.splitlines() if "warning" in l and "packed-fp32-ops" not in l]
    if warn:
        sys.stderr.write("\n".join(warn) + "\n")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", LIB, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    # the command-line driver, linked against the library (rpath $ORIGIN)
    cmd = [HIPCC, "-O2", "-std=c++17", "-I", os.path.join(ROOT, "include"),
           os.path.join(HOST, "kanjoos_run.cpp"), "-o", RUN, "-L", HERE, "-lkanjoos_amd",
           "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"kanjoos-run link failed:\n{r.stderr}")
    if verbose:
        print(f"built {LIB} and {RUN}")
    return LIB


if __name__ == "__main__":
    build()
