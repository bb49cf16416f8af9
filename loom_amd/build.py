"""Builds libloom_accel_amd.so (gfx950) in-tree with hipcc.

    python -m loom_amd.build          # or __graft_entry__.build()

Every .hip file under loom_amd/csrc is compiled for gfx950 only and linked
into loom_amd/lib/libloom_accel_amd.so, which exports loom's v2 plugin ABI
(include/loom_accel.h) and the device-resident extension
(include/loom_accel_amd.h).
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB_DIR = os.path.join(PKG, "lib")
LIB_NAME = "libloom_accel_amd.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)
OBJ_DIR = os.path.join(PKG, "_build")

ARCH = "gfx950"

# -ffp-contract=off: every fp64 rescale / norm expression rounds after each
# operation, in the reference's order (no fused multiply-add).
# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
# -amdgpu-mfma-vgpr-form: MFMA sources and results in VGPRs.  Otherwise the
# compiler places some accumulators in AGPRs and copies them to and from VGPRs
# around every MFMA of a loop; the AGPRs also count against occupancy (the fp64
# prefill attention runs 3 waves per SIMD instead of 2 with this option).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-I", os.path.join(ROOT, "include"),
    "-I", CSRC,
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build loom_amd")
    return path


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every HIP source and link the shared library; returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError("no HIP sources under " + CSRC)
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print("built", LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
