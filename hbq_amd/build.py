"""Build libhbq_amd.so (the C-ABI library) for gfx950 with hipcc, in tree.

Usage:  python -m hbq_amd.build      (or hbq_amd.build.build() from Python)

Every HIP source is compiled with -ffp-contract=off (the quantizer and GEMM
epilogues reproduce the reference's rounding step by step; a contracted
multiply-add would change results) and with packed-FP32 instructions
disabled.
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")   # the public C ABI header
OUT_DIR = os.path.join(HERE, "_lib")
LIB = os.path.join(OUT_DIR, "libhbq_amd.so")
ARCH = os.environ.get("HBQ_OFFLOAD_ARCH", "gfx950")

HIP_SOURCES = ["quant.hip", "hbq_fast.hip", "mx_fast.hip", "gemm.hip", "gemm_tile256.hip", "pack.hip", "gemm_packed.hip", "model_ops.hip"]
CXX_SOURCES = ["capi.cpp"]
COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wno-unused-function"]
HIP_FLAGS = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HBQ HIP library cannot be built")


def _compile(args):
    src, obj, flags = args
    cmd = [hipcc()] + COMMON + flags + ["-I", CSRC, "-I", INCLUDE, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose=True):
    os.makedirs(OUT_DIR, exist_ok=True)
    objdir = os.path.join(OUT_DIR, "obj")
    os.makedirs(objdir, exist_ok=True)
    jobs = []
    for s in HIP_SOURCES:
        src = os.path.join(CSRC, s)
        if os.path.exists(src):
            jobs.append((src, os.path.join(objdir, s + ".o"), HIP_FLAGS + ["-x", "hip"]))
    for s in CXX_SOURCES:
        jobs.append((os.path.join(CSRC, s), os.path.join(objdir, s + ".o"), ["-D__HIP_PLATFORM_AMD__"]))
    with ThreadPoolExecutor(max_workers=min(len(jobs), 8)) as ex:
        objs = list(ex.map(_compile, jobs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    shutil.rmtree(objdir, ignore_errors=True)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
