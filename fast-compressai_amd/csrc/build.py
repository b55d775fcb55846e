"""Build the GA-ANS HIP library for gfx950 with hipcc.

Output: fast-compressai_amd/fast_compressai/coders/lib/libgaans_w64.so
Usage:  python fast-compressai_amd/csrc/build.py   (or __graft_entry__.build())

``--phases`` builds the measurement variant instead: the same sources with
GAANS_PHASE_TIMES defined, so the kernels record phase timestamps
(gaans_debug_phases), as lib/libgaans_w64_phases.so; the package loads it
only when GAANS_PHASE_TIMES=1 is set in the environment (bench.py --phases).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)
REPO = os.path.dirname(PKG_ROOT)
SOURCES = [os.path.join(HERE, "gaans_w64.hip"), os.path.join(HERE, "gaans_host.cpp"),
           os.path.join(HERE, "rans64_host.cpp")]
OUT = os.path.join(PKG_ROOT, "fast_compressai", "coders", "lib", "libgaans_w64.so")
OUT_PHASES = os.path.join(PKG_ROOT, "fast_compressai", "coders", "lib", "libgaans_w64_phases.so")
ARCH = os.environ.get("GAANS_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Wall",
    # packed fp32 VALU ops are kept off for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(REPO, "include"),
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def build(verbose: bool = False, phases: bool = False) -> str:
    out = OUT_PHASES if phases else OUT
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    cmd = [hipcc(), *FLAGS, *(["-DGAANS_PHASE_TIMES"] if phases else []), *SOURCES, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, phases="--phases" in sys.argv))
