"""Build libkfhip.so (the gfx950 C-ABI library) in-tree with hipcc.

Usage: python kernelforge.jl_amd/build.py  (or __graft_entry__.build()).
Always recompiles; objects are built in parallel, one hipcc per source.
Also builds libkfhip_timeline.so, the scan with per-tile timestamps
(-DKF_TIMELINE) that bench.py --timeline loads.
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
# instrumented scan (per-tile timestamps, KF_TIMELINE) for bench.py --timeline
TIMELINE_LIB = os.path.join(HERE, "libkfhip_timeline.so")
TIMELINE_SOURCES = ["kf_api.hip", "kf_scan.hip", "kf_reduce.hip"]
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


def _compile(src, extra=()):
    tag = "_tl" if extra else ""
    obj = os.path.join(OBJ, src.replace(".hip", f"{tag}.o"))
    cmd = [HIPCC, *FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def _link(objs, lib):
    tmp = lib + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib)


def build_timeline(verbose=True):
    """libkfhip_timeline.so: the scan with per-tile timestamps (KF_TIMELINE)."""
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(TIMELINE_SOURCES)) as ex:
        objs = list(ex.map(lambda s: _compile(s, ("-DKF_TIMELINE",)), TIMELINE_SOURCES))
    _link(objs, TIMELINE_LIB)
    if verbose:
        print(f"built {TIMELINE_LIB}")
    return TIMELINE_LIB


def build(verbose=True, timeline=True):
    os.makedirs(OBJ, exist_ok=True)
    jobs = [(s, ()) for s in SOURCES] + ([(s, ("-DKF_TIMELINE",)) for s in TIMELINE_SOURCES] if timeline else [])
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        objs = list(ex.map(lambda j: _compile(*j), jobs))
    _link(objs[:len(SOURCES)], LIB)
    if timeline:
        _link(objs[len(SOURCES):], TIMELINE_LIB)
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
        if timeline:
            print(f"built {TIMELINE_LIB}")
        print(f"built {DRIVER}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
