"""Builds librew_mi355x.so in-tree with hipcc for gfx950.

Every source under rew_amd/csrc is compiled to an object file under
rew_amd/_build/ (in parallel), then linked into rew_amd/librew_mi355x.so.
The library is the product: Python only loads it through ctypes.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "librew_mi355x.so"
ARCH = os.environ.get("REW_MI355X_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
          "-Wno-unused-variable", "-Wno-unused-parameter",
          # host code: no FMA contraction, so generators and host math are
          # reproducible bit for bit
          "-ffp-contract=off"]
DEVICE = [f"--offload-arch={ARCH}", "-munsafe-fp-atomics",
          # keep the compiler from emitting packed-fp32 VALU ops
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    if src.suffix == ".hip":
        cmd = [HIPCC, *COMMON, *DEVICE, "-x", "hip", "-c", str(src), "-o", str(obj)]
    else:
        cmd = [HIPCC, *COMMON, "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
               "-x", "c++", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compiles every csrc file and links the shared library; returns its path."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; cannot build librew_mi355x.so")
    BUILD.mkdir(exist_ok=True)
    srcs = sorted([*CSRC.glob("*.cpp"), *CSRC.glob("*.hip")])
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", str(tmp),
           *map(str, objs), "-L/opt/rocm/lib", "-lhiprtc", "-ldl", "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
