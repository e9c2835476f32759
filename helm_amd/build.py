"""Builds libhelm_amd.so (all HIP sources under helm_amd/csrc) for gfx950.

Usage: python -m helm_amd.build [--incremental]

Every .hip file is compiled to an object with hipcc (in parallel), then the
objects are linked into helm_amd/libhelm_amd.so, the library the ctypes shim
(helm_amd/_native.py) loads.  The library is built in-tree so it travels with
the source tree; it is listed in .gitignore.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libhelm_amd.so"
ARCH = os.environ.get("HELM_AMD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
    # no packed-fp32 instructions in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs: the decode kernel rescales them
    # with vector ALU ops, which cannot address AGPRs
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    # atomics as written: the decode kernel's block claims are issued by one
    # lane and their results read a step later; the atomic optimizer would
    # broadcast each result right after the atomic, a wait on every load
    # in flight
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build libhelm_amd.so")


def _deps_mtime() -> float:
    files = list(CSRC.glob("*.h")) + [ROOT / "include" / "helm_amd.h"]
    return max(f.stat().st_mtime for f in files)


def _compile(hipcc: str, src: Path, obj: Path) -> None:
    cmd = [hipcc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


CPU_SRCS = [PKG / "cpu" / "gemv.cpp", PKG / "cpu" / "attn.cpp"]
CPU_LIB = PKG / "libhelm_cpu.so"
# host code only: no -march (the library runs on another machine's CPU); the
# AVX2 / AVX-512 paths carry their own target attributes and are chosen at run
# time from CPUID
CPU_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", "-fopenmp", "-Wall",
             f"-I{ROOT / 'include'}"]


def build_cpu(verbose: bool = True) -> Path:
    """Compiles the host-CPU sources (helm_amd/cpu: the fp16 GEMV and the
    streaming attention of HELM's CPU stages) into libhelm_cpu.so with g++;
    returns its path."""
    gxx = shutil.which("g++") or shutil.which("c++")
    if not gxx:
        raise RuntimeError("g++ not found: needed for libhelm_cpu.so")
    tmp = CPU_LIB.with_suffix(".so.tmp")
    res = subprocess.run([gxx, *CPU_FLAGS, *map(str, CPU_SRCS), "-o", str(tmp)],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed for libhelm_cpu.so:\n{res.stderr}")
    os.replace(tmp, CPU_LIB)
    if verbose:
        print(f"[helm_amd.build] wrote {CPU_LIB}", flush=True)
    return CPU_LIB


def build(incremental: bool = False, jobs: int | None = None, verbose: bool = True) -> Path:
    """Compiles every HIP source and links libhelm_amd.so, and builds
    libhelm_cpu.so; returns the path of libhelm_amd.so."""
    build_cpu(verbose=verbose)
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    deps = _deps_mtime()
    todo = []
    for src in sources:
        obj = BUILD / (src.stem + ".o")
        stale = (not obj.exists() or obj.stat().st_mtime < max(src.stat().st_mtime, deps))
        if not incremental or stale:
            todo.append((src, obj))
    jobs = jobs or min(len(todo) or 1, max(1, min(16, os.cpu_count() or 4)))
    if verbose and todo:
        print(f"[helm_amd.build] compiling {len(todo)} HIP sources for {ARCH} "
              f"({jobs} jobs)", flush=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda t: _compile(hipcc, *t), todo))
    objs = [str(BUILD / (s.stem + ".o")) for s in sources]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs,
           "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[helm_amd.build] wrote {LIB}", flush=True)
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--incremental", action="store_true",
                    help="recompile only sources newer than their objects")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    a = ap.parse_args()
    build(incremental=a.incremental, jobs=a.jobs)


if __name__ == "__main__":
    main()
