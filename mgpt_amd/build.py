"""Builds the native libraries in-tree (they travel with the repository).

  mgpt_amd/lib/libmgpt_moe.so      HIP kernels + C ABI (include/mgpt_moe.h), gfx950
  mgpt_amd/lib/libmgpt_workload.so seeded synthetic-input generator (host C)

Usage: python -m mgpt_amd.build  (or __graft_entry__.build()).
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
LIB = os.path.join(HERE, "lib")
OBJ = os.path.join(HERE, "_build")

HIP_SOURCES = ["router.hip", "dispatch.hip", "gemm.hip", "gemm_dma.hip", "gemm_decode.hip", "combine.hip",
               "pack.hip", "backward.hip", "wgrad.hip", "moe_capi.hip", "checkpoint.cpp"]
ARCH = os.environ.get("MGPT_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off: the router must round every product and sum separately
# to reproduce the reference's bits.  Packed-fp32 instructions are disabled.
HIPCC_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-Wall", "-Wno-unused-function", "-I" + os.path.join(ROOT, "include")]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the MI355X kernels cannot be built")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n"
                           f"{r.stdout}\n{r.stderr}")
    return r


def build_hip(verbose: bool = False) -> str:
    os.makedirs(LIB, exist_ok=True)
    os.makedirs(OBJ, exist_ok=True)
    hipcc = _hipcc()
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=min(8, len(cmds))) as ex:
        for r in ex.map(_run, cmds):
            if verbose and r.stderr:
                print(r.stderr, file=sys.stderr)
    out = os.path.join(LIB, "libmgpt_moe.so")
    tmp = out + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    return out


def build_workload() -> str:
    os.makedirs(LIB, exist_ok=True)
    out = os.path.join(LIB, "libmgpt_workload.so")
    _run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", "-fPIC", "-shared", "-o", out,
          os.path.join(CSRC, "workload_gen.c"), "-lm"])
    return out


def build_all(verbose: bool = False) -> None:
    build_workload()
    build_hip(verbose)


if __name__ == "__main__":
    build_all(verbose=True)
    print("built", os.listdir(LIB))
