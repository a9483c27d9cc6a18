"""Build recipe for libmoeq.so (gfx950) and the oracle's C library.

``python -m robustgemq_amd.build`` compiles every ``csrc/*.hip`` file with
hipcc for gfx950 into ``robustgemq_amd/_build/*.o`` (in parallel) and links
``robustgemq_amd/libmoeq.so`` in-tree, so the library travels with the source
tree to the GPU machine.  No torch extension machinery is involved: the
library exposes a C ABI (include/moeq.h) loaded with ctypes.
"""

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libmoeq.so")
ARCH = os.environ.get("MOEQ_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-mcode-object-version=5",
    "-fno-gpu-flush-denormals-to-zero",
    # packed fp32 VALU forms are disabled on this platform
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unused-lambda-capture",
]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmoeq.so)")


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    out = "\n".join(l for l in p.stdout.splitlines() if "not a recognized feature" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build_lib(jobs=None, verbose=False):
    hipcc = _hipcc()
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]

    def compile_one(src):
        obj = os.path.join(OBJ, os.path.basename(src)[:-4] + ".o")
        out = _run([hipcc, *HIPCC_FLAGS, *inc, "-c", src, "-o", obj])
        if verbose and out.strip():
            print(out)
        return obj

    jobs = jobs or min(8, os.cpu_count() or 1, len(srcs))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


def build_oracle():
    """Compile the oracle's C restatement (test infrastructure) with gcc."""
    odir = os.path.join(ROOT, "oracle")
    out = os.path.join(odir, "_build", "liboracle.so")
    os.makedirs(os.path.dirname(out), exist_ok=True)
    _run(["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-std=c99",
          "-o", out, os.path.join(odir, "router_exact.c"), "-lm"])
    return out


if __name__ == "__main__":
    print(build_lib(verbose="-v" in sys.argv))
    print(build_oracle())
