"""Builds libprichs_hip.so in-tree with hipcc for gfx950.

Every .hip file under csrc/ is compiled to an object in parallel, then linked
into prichs_amd/libprichs_hip.so.  No JIT cache and no site-packages install:
the library sits next to this file so it travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libprichs_hip.so")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libprichs_hip.so)")


COMMON_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-Wall",
    # Keep hipcc from forming packed-FP32 instructions (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_host(verbose)
    return LIB


HOST = os.path.join(HERE, "host")
HOST_LIB = os.path.join(HERE, "libprichs_host.so")
HOST_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "test_gpu_model_engine.cpp")
HOST_TEST_BIN = os.path.join(ROOT, "tests", "cpp", "test_gpu_model_engine")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def _gxx(args, what):
    cxx = os.environ.get("CXX", "g++")
    r = subprocess.run([cxx, *args], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{r.stderr}")


def build_host(verbose: bool = False) -> str:
    """The C++ host mirror of GpuModelEngine (libprichs_host.so, over the C ABI
    of libprichs_hip.so) and its C++ test program; plain host C++ with the HIP
    runtime, so g++ builds it.  rpaths are relative ($ORIGIN) so both travel
    with the tree."""
    flags = ["-std=c++17", "-O2", "-Wall", "-D__HIP_PLATFORM_AMD__",
             "-I", os.path.join(ROCM, "include"), "-I", os.path.join(ROOT, "include"), "-I", HOST]
    rocm_lib = ["-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"]
    _gxx([*flags, "-fPIC", "-shared", os.path.join(HOST, "gpu_model_engine.cpp"), "-L", HERE,
          "-lprichs_hip", *rocm_lib, "-Wl,-rpath,$ORIGIN", "-o", HOST_LIB], "libprichs_host.so")
    _gxx([*flags, HOST_TEST_SRC, "-L", HERE, "-lprichs_host", "-lprichs_hip", *rocm_lib,
          "-Wl,-rpath,$ORIGIN/../../prichs_amd", "-o", HOST_TEST_BIN], "test_gpu_model_engine")
    if verbose:
        print(f"built {HOST_LIB} and {HOST_TEST_BIN}")
    return HOST_LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
