"""Build step for libhipgemm.so (the C ABI + gfx950 kernels).

``python -m hipgemm_amd.build`` compiles every hipgemm_amd/csrc/*.hip with
hipcc for gfx950 (in parallel, one object per file under
hipgemm_amd/_build/), then links them into hipgemm_amd/libhipgemm.so,
in-tree, so the library travels with the source tree.  It also builds
hipgemm_amd/libhipgemm_probe.so from probe/mfma_ceiling.hip, the MFMA ceiling
probe that bench.py reports beside the GEMM.  No GPU is needed to
build.
"""
from __future__ import annotations

import glob
import os
import shlex
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
CSRC = os.path.join(PKG, "csrc")
SRCS = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
OBJDIR = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libhipgemm.so")
# Measurement-only probe (bench.py's MFMA ceiling), a library of its own so
# that nothing of it is linked into libhipgemm.so.
PROBE_SRC = os.path.join(PKG, "probe", "mfma_ceiling.hip")
PROBE_LIB = os.path.join(PKG, "libhipgemm_probe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-FP32 instructions are disabled for every HIP build (the compiler
# otherwise forms v_pk_*_f32 from scalar float code).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]
_NOISE = "is not a recognized feature for this target"


def compile_cmd(src: str, obj: str) -> list:
    return [HIPCC, *HIP_FLAGS, "-c", f"-I{INCLUDE}", f"-I{CSRC}", src, "-o",
            obj]


def link_cmd(objs, out: str) -> list:
    return [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o",
            out]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(shlex.quote(c) for c in cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if _NOISE not in l)
    if res.returncode != 0:
        raise RuntimeError(f"{cmd[0]} failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int = 0) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    objs = [os.path.join(OBJDIR, os.path.basename(s)[:-4] + ".o") for s in SRCS]
    jobs = jobs or min(len(SRCS), max(1, os.cpu_count() or 1), 8)
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(lambda so: _run(compile_cmd(*so), verbose),
                      zip(SRCS, objs)))
    tmp = LIB + ".tmp"
    _run(link_cmd(objs, tmp), verbose)
    os.replace(tmp, LIB)
    tmp = PROBE_LIB + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", f"-I{INCLUDE}", PROBE_SRC, "-o", tmp],
         verbose)
    os.replace(tmp, PROBE_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
