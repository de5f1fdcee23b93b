"""Build step for libhipgemm.so (the C ABI + gfx950 kernels).

``python -m hipgemm_amd.build`` compiles hipgemm_amd/csrc/hipgemm.hip with
hipcc for gfx950 into hipgemm_amd/libhipgemm.so, in-tree, so the library
travels with the source tree.  No GPU is needed to build.
"""
from __future__ import annotations

import os
import shlex
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
SRC = os.path.join(PKG, "csrc", "hipgemm.hip")
LIB = os.path.join(PKG, "libhipgemm.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-FP32 instructions are disabled for every HIP build (the compiler
# otherwise forms v_pk_*_f32 from scalar float code).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


def hipcc_cmd(src: str = SRC, out: str = LIB, extra=()) -> list:
    return [HIPCC, *HIP_FLAGS, "-shared", f"-I{INCLUDE}", src, "-o", out,
            *extra]


def build(verbose: bool = False) -> str:
    cmd = hipcc_cmd()
    if verbose:
        print(" ".join(shlex.quote(c) for c in cmd), flush=True)
    tmp = LIB + ".tmp"
    cmd[cmd.index(LIB)] = tmp
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
