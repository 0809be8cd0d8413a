"""Builds libtwd_head.so in-tree with hipcc for gfx950.

    python turbo-winfare-dense_amd/build.py          # compile every source, link the library

Every call compiles from scratch (seconds per file); objects go to _build/ beside this file and
the library to libtwd_head.so beside this file, where tests, bench.py and the GPU box load it.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libtwd_head.so")
SOURCES = ["csrc/head.hip", "csrc/select.hip", "csrc/verify.hip", "csrc/host.cpp", "csrc/g4dense_api.cpp",
           "csrc/container.cpp", "csrc/generator.cpp", "csrc/probe.hip"]
ARCH = os.environ.get("TWD_OFFLOAD_ARCH", "gfx950")

# Packed-fp32 VALU forms are kept out of the code object: hipcc would otherwise pair fp32 adds
# and multiplies into v_pk_* instructions on its own. MFMA results stay in ordinary VGPRs: the
# head kernels read every accumulator back on the VALU, and accumulation registers would cost
# a copy per read.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                "-mllvm", "-amdgpu-mfma-vgpr-form"]
COMMON = ["-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall",
          f"--offload-arch={ARCH}", "-I" + os.path.join(ROOT, "include"),
          "-I" + os.path.join(HERE, "csrc")]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: str, out_dir: str) -> str:
    obj = os.path.join(out_dir, os.path.basename(src) + ".o")
    cmd = [hipcc(), "-x", "hip", "-c", os.path.join(HERE, src), "-o", obj] + COMMON + DEVICE_FLAGS
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    out_dir = os.path.join(HERE, "_build")
    os.makedirs(out_dir, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(4, len(SOURCES))) as ex:
        objs = list(ex.map(lambda s: _compile(s, out_dir), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp] + objs
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
