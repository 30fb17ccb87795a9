"""Build libgrimoire_moe.so (gfx950) in-tree with hipcc.

    python -m grimoire_amd.build            # or grimoire_amd.build.build()
    python -m grimoire_amd.build --timing   # the phase-stamp build (below)

Each HIP source compiles to an object in grimoire_amd/_build/, then one
shared library grimoire_amd/libgrimoire_moe.so is linked.  The built
library travels with the source tree; nothing is installed.

--timing builds the same sources with GRIM_TIMING into
grimoire_amd/_timing/libgrimoire_moe.so: the decode kernels then stamp the
real-time counter at their phase boundaries into a buffer the caller hands
over (grim_timing_set), which grimoire_amd.phase_timeline reads.  It is a
measurement build, never the product library.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libgrimoire_moe.so"
OBJ = PKG / "_build"

SOURCES = ["router.hip", "gemv.hip", "gemv_f0.hip", "gemv_f3.hip", "gemv_f4.hip", "gemv_f6.hip",
           "gemv_f64.hip", "dispatch.hip", "gemm.hip", "gemm_i8.hip", "ingest.hip",
           "tiered.hip", "elementwise.hip", "gemv_grouped.hip", "gemv_mx.hip", "api.cpp", "forward.cpp", "heat.cpp"]
# host-only sources (x86 intrinsics, threads): the C++ compiler, not hipcc
HOST_SOURCES = ["cpu_experts.cc"]
CXX = os.environ.get("CXX", "g++")
HOST_FLAGS = ["-O3", "-std=c++20", "-fPIC", "-fvisibility=hidden", "-ffp-contract=off", "-pthread",
              "-Wall", "-I" + str(PKG.parent / "include")]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # no packed fp32 instructions (v_pk_fma_f32 and friends) anywhere
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-pass-failed",
]


def _compile(src: str) -> Path:
    obj = OBJ / (Path(src).stem + ".o")
    cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def _compile_host(src: str) -> Path:
    obj = OBJ / (Path(src).stem + ".o")
    cmd = [CXX, *HOST_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{CXX} failed for {src}:\n{r.stderr}")
    if r.stderr.strip():
        print(r.stderr, file=sys.stderr)
    return obj


def build_timing(verbose: bool = True) -> Path:
    """The GRIM_TIMING build into grimoire_amd/_timing/ (objects in
    grimoire_amd/_build_timing/)."""
    global OUT, OBJ, FLAGS, HOST_FLAGS
    saved = OUT, OBJ, FLAGS, HOST_FLAGS
    OUT, OBJ = PKG / "_timing" / "libgrimoire_moe.so", PKG / "_build_timing"
    FLAGS, HOST_FLAGS = FLAGS + ["-DGRIM_TIMING"], HOST_FLAGS + ["-DGRIM_TIMING"]
    try:
        OUT.parent.mkdir(exist_ok=True)
        return build(verbose)
    finally:
        OUT, OBJ, FLAGS, HOST_FLAGS = saved


def build(verbose: bool = True) -> Path:
    """Compile every source and link the shared library; returns its path."""
    OBJ.mkdir(exist_ok=True)
    jobs = min(len(SOURCES), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES)) + list(ex.map(_compile_host, HOST_SOURCES))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-pthread", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build_timing() if "--timing" in sys.argv[1:] else build()
