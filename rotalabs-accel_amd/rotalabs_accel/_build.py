"""Build librotaccel.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python -m rotalabs_accel._build        (from rotalabs-accel_amd/)

Every .hip file under rotalabs-accel_amd/csrc is compiled for gfx950 only and
linked into rotalabs_accel/_lib/librotaccel.so. Flags that matter:

* ``-Xclang -target-feature -Xclang -packed-fp32-ops`` keeps the compiler from
  emitting packed-fp32 VALU instructions (v_pk_{add,mul,fma}_f32);
* ``-fhip-fp32-correctly-rounded-divide-sqrt`` and no fast-math: the weight
  quantiser and RMSNorm depend on IEEE fp32 division / square root;
* ``-mllvm -amdgpu-kernarg-preload-count=16``: the first kernel-argument
  dwords (as many as the free user SGPRs hold, 13 for these kernels) arrive in
  SGPRs at wave launch instead of through scalar loads. The decode kernels'
  first weight loads wait for their arguments; each round trip of scalar
  argument loads delays every wave's start. The argument lists put what the
  kernels need first (pointers, sizes) ahead of the output pointer.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
PROJ_DIR = os.path.dirname(PKG_DIR)                 # rotalabs-accel_amd/
REPO_DIR = os.path.dirname(PROJ_DIR)
CSRC = os.path.join(PROJ_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
BUILD_DIR = os.path.join(PROJ_DIR, "_build")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_PATH = os.path.join(LIB_DIR, "librotaccel.so")

ARCH = "gfx950"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build librotaccel.so)")


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-fno-fast-math",
        "-fhip-fp32-correctly-rounded-divide-sqrt",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-mllvm", "-amdgpu-kernarg-preload-count=16",
        "-Wno-unused-command-line-argument",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
    ]


def _compile_one(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    cmd = [_hipcc(), *compile_flags(), "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every csrc/*.hip for gfx950 and link librotaccel.so. Returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile_one, sources))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
