"""Build libkfhip.so (the gfx950 C-ABI library) in-tree with hipcc.

Usage: python kernelforge.jl_amd/build.py  (or __graft_entry__.build()).
Always recompiles; objects are built in parallel, one hipcc per source.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libkfhip.so")
DRIVER = os.path.join(HERE, "kf_driver")
SOURCES = ["kf_api.hip", "kf_scan.hip", "kf_reduce.hip", "kf_reduce_dims.hip", "kf_matvec.hip", "kf_copy.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fno-strict-aliasing",
    "-ffp-contract=off",
    # packed FP32 instructions are kept out of every kernel on this hardware pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(REPO, "include"),
]


def _compile(src):
    obj = os.path.join(OBJ, src.replace(".hip", ".o"))
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose=True):
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    # the plain C-ABI driver (host code only: g++ against the HIP runtime)
    cmd = ["g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I", "/opt/rocm/include",
           "-I", os.path.join(REPO, "include"), os.path.join(CSRC, "kf_driver.cpp"), "-o", DRIVER + ".tmp",
           "-L", HERE, "-lkfhip", "-L", "/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN",
           "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"kf_driver build failed:\n{r.stderr}")
    os.replace(DRIVER + ".tmp", DRIVER)
    if verbose:
        print(f"built {LIB}")
        print(f"built {DRIVER}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
