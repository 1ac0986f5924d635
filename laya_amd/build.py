"""Builds liblaya_hip.so in-tree for gfx950 with hipcc (no CMake, no JIT cache).

    python -m laya_amd.build        # or laya_amd.build.build() from Python

Every source is compiled as HIP for gfx950 only, with packed-fp32 instruction selection turned off
(-Xclang -target-feature -Xclang -packed-fp32-ops); the objects go to laya_amd/_build and the
shared library to laya_amd/liblaya_hip.so, which travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "liblaya_hip.so")
SOURCES = ["gemm.hip", "norm.hip", "attention.hip", "elementwise.hip", "optim.hip", "objective.hip", "readout.hip", "capi.cpp", "model.cpp"]
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-Wall", "-Wno-unused-function", "-Wno-unused-result"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return "hipcc"


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that note is expected.
    lines = [ln for ln in r.stdout.splitlines() if "packed-fp32-ops" not in ln]
    return r.returncode, "\n".join(lines)


def build(verbose: bool = False, jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = _hipcc()

    def compile_one(src):
        obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
        cmd = [hipcc, "-x", "hip", *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
        rc, out = _run(cmd)
        if rc != 0:
            raise RuntimeError(f"compiling {src} failed:\n{out}")
        if verbose and out.strip():
            print(out)
        return obj

    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(SOURCES)))) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    rc, out = _run([hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp, *objs])
    if rc != 0:
        raise RuntimeError(f"linking liblaya_hip.so failed:\n{out}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print("built", path)
