"""Build libsparton_hip.so (gfx950) in-tree with hipcc.

Usage: python -m sparton_amd.build   (or sparton_amd.build.build_library()).
Each source is compiled to an object in parallel, then linked into one shared
library next to this file. No cmake/ninja; the only tool is hipcc.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libsparton_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
TORCH_LIB_NAME = "libsparton_torch.so"   # the eager torch ops (C++ autograd), on the C ABI above
TORCH_LIB_PATH = os.path.join(HERE, TORCH_LIB_NAME)
SOURCES = ["sparton_fwd.hip", "sparton_bwd.hip", "sparton_transform.hip", "sparton_loss.hip",
           "sparton_probe.hip", "sparton_capi.cpp"]
ARCH = os.environ.get("SPARTON_OFFLOAD_ARCH", "gfx950")

# Packed-fp32 VALU ops are disabled on purpose: hipcc would otherwise emit
# v_pk_{add,mul,fma}_f32 from plain float code, and those are avoided on these boxes.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall",
                "-Wno-unused-result"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm at /opt/rocm)")


def _compile(hipcc: str, src: str, obj: str) -> None:
    cmd = [hipcc, *COMMON_FLAGS]
    if src.endswith(".hip"):
        cmd += [f"--offload-arch={ARCH}", *DEVICE_FLAGS, "-x", "hip"]
    cmd += ["-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build_library(verbose: bool = False) -> str:
    hipcc = _hipcc()
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        list(ex.map(lambda so: _compile(hipcc, *so), zip(SOURCES, objs)))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    build_torch_ops(verbose)
    return LIB_PATH


def build_torch_ops(verbose: bool = False) -> str:
    """libsparton_torch.so: the sparton_eager torch ops (csrc/sparton_torch.cpp), a host-only
    C++ library compiled with g++ against libtorch and linked to libsparton_hip.so, which it
    finds next to itself (rpath $ORIGIN)."""
    import torch
    tdir = os.path.dirname(torch.__file__)
    cxx = os.environ.get("CXX", "g++")
    tmp = TORCH_LIB_PATH + ".tmp"
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden", "-Wall",
           "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           "-I", os.path.join(tdir, "include"),
           "-I", os.path.join(tdir, "include", "torch", "csrc", "api", "include"),
           "-I", "/opt/rocm/include",
           os.path.join(CSRC, "sparton_torch.cpp"), "-o", tmp,
           "-L", os.path.join(tdir, "lib"), "-ltorch", "-ltorch_cpu", "-lc10", "-lc10_hip",
           "-ltorch_hip", "-lhipblaslt", "-L", HERE, "-lsparton_hip",
           f"-Wl,-rpath,{os.path.join(tdir, 'lib')}", "-Wl,-rpath,$ORIGIN"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, TORCH_LIB_PATH)
    if verbose:
        print(f"built {TORCH_LIB_PATH}")
    return TORCH_LIB_PATH


if __name__ == "__main__":
    build_library(verbose=True)
    sys.exit(0)
