"""Builds HELM's own fp16 GEMV (helm/kernels/fp16_gemv.cpp) from the reference
tree into oracle/_ref/ — TEST INFRASTRUCTURE ONLY (a reference for the GEMV
tests and the CPU baseline of the GEMV leg, never part of the product).

One g++ command on the one source file where it lies, against the installed
torch (the file is a torch extension: torch/extension.h + pybind11).  HELM
builds it with torch.utils.cpp_extension.load and -march=native
(helm/kernels/__init__.py:41-47); here the ISA flags are spelled out
(-mavx2 -mf16c -mfma, the instructions the file uses) because the module runs
on another machine's CPU than the one that builds it.  Nothing is built when
the reference tree is absent.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from pathlib import Path

REF_SRC = Path("/root/reference/helm/kernels/fp16_gemv.cpp")
OUT_DIR = Path(__file__).resolve().parent / "_ref"
MODULE = "helm_ref_fp16_gemv"
OUT = OUT_DIR / f"{MODULE}.so"


def build(verbose: bool = True) -> Path | None:
    if not REF_SRC.exists():
        if verbose:
            print(f"[oracle.build_ref] {REF_SRC} absent: nothing built", flush=True)
        return None
    import torch
    import torch.utils.cpp_extension as ce
    OUT_DIR.mkdir(exist_ok=True)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O3", "-std=c++17", "-fPIC", "-shared", "-mavx2", "-mf16c", "-mfma",
           "-ffast-math", "-fopenmp", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           f"-DTORCH_EXTENSION_NAME={MODULE}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           *[f"-I{p}" for p in ce.include_paths()], f"-I{sysconfig.get_paths()['include']}",
           str(REF_SRC), "-o", str(OUT) + ".tmp",
           *[f"-L{p}" for p in ce.library_paths()],
           *[f"-Wl,-rpath,{p}" for p in ce.library_paths()],
           "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-fopenmp"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed for {REF_SRC}:\n{res.stderr[-4000:]}")
    os.replace(str(OUT) + ".tmp", OUT)
    if verbose:
        print(f"[oracle.build_ref] wrote {OUT}", flush=True)
    return OUT


def load():
    """The built module (import torch first), or None when not built."""
    if not OUT.exists():
        return None
    import importlib.util
    spec = importlib.util.spec_from_file_location(MODULE, OUT)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


if __name__ == "__main__":
    sys.exit(0 if build() is not None else 1)
