"""Builds lib/libktmi.so from csrc/ with hipcc for gfx950 (cross-compiles without a GPU).

    python kt-prefill-lend_amd/build.py [-j N]
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "lib" / "libktmi.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("KTMI_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    # no packed fp32 (v_pk_*_f32) code generation
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    # the first kernel arguments arrive in SGPRs with the dispatch instead of by a scalar load
    # (decode launches 0.1-0.5 us shorter each on MI355X)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]
CXX_FLAGS = ["-O3", "-fPIC", "-std=c++17", "-pthread", "-ffp-contract=off", "-Wall"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def build(jobs: int = 8, verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    hips = sorted(CSRC.glob("*.hip"))
    cpps = sorted(CSRC.glob("*.cpp"))
    cmds = []
    objs = []
    for src in hips:
        o = OBJ / (src.stem + ".o")
        cmds.append([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(o)])
        objs.append(o)
    for src in cpps:
        o = OBJ / (src.stem + ".cpp.o")
        cmds.append(["g++", *CXX_FLAGS, "-c", str(src), "-o", str(o)])
        objs.append(o)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for r in ex.map(_run, cmds):
            if verbose and r.stderr.strip():
                print(r.stderr, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=8)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.v))
