"""Build the C-ABI library nwc_amd/lib/nwc_ops.so for MI355X (gfx950) with hipcc.

usage: python -m nwc_amd.build [--arch gfx950] [--jobs N] [--verbose]

Counterpart of the reference's nvcc build (nwc/build.py:34-46).  Every source under nwc_amd/csrc is compiled to
an object in nwc_amd/_build (in parallel), then linked into one shared library.  hipcc cross-compiles, so this
runs on a machine without a GPU.
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
TARGET_DIR = os.path.join(HERE, "lib")
TARGET = os.path.join(TARGET_DIR, "nwc_ops.so")
SOURCES = ["encode.cpp", "abi.cpp", "kern_prefix.hip", "kern_fixed.hip", "kern_misc.hip", "kern_gemm.hip"]
# -packed-fp32-ops: no v_pk_*_f32 anywhere (hipcc's host pass warns that it does not know the feature)
# -amdgpu-kernarg-preload-count: gfx950 loads a kernel's leading scalar arguments into SGPRs before its first
# instruction (kernels that take them, k_layout0p); kernels whose first argument is a struct keep reading theirs
COMMON = ["-O3", "-fPIC", "-std=c++17", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-mllvm", "-amdgpu-kernarg-preload-count=8", "-I" + CSRC, "-I" + os.path.join(ROOT, "include")]


def find_hipcc():
    for c in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    raise SystemExit("hipcc not found")


def _compile(hipcc, arch, src, verbose):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc, "--offload-arch=" + arch, *COMMON, "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l]
    if r.returncode:
        raise RuntimeError(f"hipcc failed on {src}:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs))
    return obj


def build(arch="gfx950", jobs=None, verbose=False):
    hipcc = find_hipcc()
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(TARGET_DIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, arch, s, verbose), SOURCES))
    tmp = TARGET + ".tmp"
    cmd = [hipcc, "--offload-arch=" + arch, "-shared", "-fPIC", "-pthread", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, TARGET)
    if verbose:
        print("built:", TARGET)
    return TARGET


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--arch", default="gfx950")
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args()
    try:
        build(a.arch, a.jobs, a.verbose)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
