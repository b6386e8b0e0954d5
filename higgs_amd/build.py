"""Build libhiggs_hip.so (the C-ABI library) in-tree with hipcc for gfx950.

    python -m higgs_amd.build          # or: python higgs_amd/build.py

Each ``csrc/*.hip`` is compiled to an object in ``higgs_amd/_build`` (in
parallel), then linked into ``higgs_amd/libhiggs_hip.so``. The C++ host API
(``host/higgs.cpp``) is then built over it into ``higgs_amd/libhiggs.so``. hipcc cross-compiles
without a GPU, so this runs anywhere the ROCm toolchain is installed.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libhiggs_hip.so")
HOST = os.path.join(HERE, "host")
HOST_LIB = os.path.join(HERE, "libhiggs.so")
ARCH = os.environ.get("HGK_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off: products and sums are rounded separately, exactly as the
# separately materialised MLX ops they reproduce (no silent FMA contraction).
# The packed-FP32 feature is switched off for the device pass.
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(cc: str, src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [cc, *CFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(ln for ln in r.stderr.splitlines() if noise not in ln)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    cc = hipcc()
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    workers = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(cc, s), srcs))
    tmp = LIB + ".tmp"
    r = subprocess.run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_host(verbose)
    return LIB


def build_host(verbose: bool = True) -> str:
    """libhiggs.so: the C++ host API (host/higgs.hpp) over libhiggs_hip.so."""
    cxx = os.environ.get("CXX") or shutil.which("g++") or "g++"
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    srcs = sorted(glob.glob(os.path.join(HOST, "*.cpp")))
    tmp = HOST_LIB + ".tmp"
    cmd = [cxx, "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra",
           "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(os.path.dirname(HERE), "include"),
           "-I", os.path.join(rocm, "include"), *srcs, "-o", tmp,
           "-L", HERE, "-lhiggs_hip", "-L", os.path.join(rocm, "lib"), "-lamdhip64",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{os.path.join(rocm, 'lib')}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host library build failed:\n{r.stderr}")
    os.replace(tmp, HOST_LIB)
    if verbose:
        print(f"built {HOST_LIB}")
    return HOST_LIB


if __name__ == "__main__":
    build()
